// libfirewing_hip_moe: the sparse-MoE block hot path for MI355X (gfx950)
// behind the C ABI of include/firewing_hip_moe.h.
//
// Stateless entry points (linear, SwiGLU, sigmoid, top-k, route, expert) copy
// host buffers in, run exact-order kernels and copy out. The resident context
// keeps every layer's weights in HBM and runs a whole block, or a whole
// 48-layer decode step, as one persistent launch (fw_decode.h).
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "../../include/firewing_hip_moe.h"
#include "fw_decode.h"
#include "fw_device.h"
#include "fw_hyper.h"
#include "fw_lm_head.h"
#include "fw_zstd_host.h"
#include "fw_numerics.h"
#include "fw_prefill.h"
#include "fw_safetensors.h"
#include "fw_synth.h"

using namespace fw;

// The decode kernels are instantiated in fw_decode_kernels.hip.
namespace fw {
#define FW_EXTERN(NT, MBH, MBI, TK) \
    extern template __global__ void k_moe_decode<NT, MBH, MBI, TK>(const DecodeParams*, uint32_t);
FW_DECODE_VARIANTS(FW_EXTERN)
FW_DECODE_VARIANTS_ONE_TOKEN(FW_EXTERN)
#undef FW_EXTERN
}  // namespace fw

// ---- error reporting ------------------------------------------------------------------

namespace {

thread_local std::string g_last_error;

bool fail(const std::string& message) {
    g_last_error = message;
    return false;
}

struct HipError {
    std::string message;
};

void check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw HipError{std::string(what) + ": " + hipGetErrorString(status)};
    }
}

template <typename F>
bool guarded(F&& body) {
    try {
        return body();
    } catch (const HipError& e) {
        return fail(e.message);
    } catch (const std::bad_alloc&) {
        return fail("host allocation failed");
    } catch (const std::exception& e) {
        return fail(e.what());
    } catch (...) {
        return fail("unexpected failure");
    }
}

// Host copy of the 2^(i/32) table (same constants as c_exp2_table).
const uint64_t kExp2TableHost[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

// RAII device buffer for the stateless entry points.
struct DeviceBuffer {
    void* ptr = nullptr;
    explicit DeviceBuffer(size_t bytes) {
        if (bytes) check(hipMalloc(&ptr, bytes), "hipMalloc");
    }
    ~DeviceBuffer() {
        if (ptr) (void)hipFree(ptr);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    template <typename T>
    T* as() const {
        return static_cast<T*>(ptr);
    }
};

void upload(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes) check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
}
void download(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes) check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
}

}  // namespace

// ---- standalone kernels -----------------------------------------------------------------

namespace fw {

// out[t][r] = bf16(tree32(W[r,:], x[t,:])) for NT tokens; 4 rows per wave,
// 16 rows per 256-thread block; x staged in LDS as f32 (dynamic shared). The
// row is swept in chunks of 32 blocks, each chunk's loads issued together.
template <int NT>
__global__ void __launch_bounds__(256) k_linear_tree32(const uint16_t* __restrict__ w,
                                                       const uint16_t* __restrict__ x, int rows,
                                                       int K, uint16_t* __restrict__ out) {
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < NT * K; i += blockDim.x) xs[i] = from_bf16(x[i]);
    __syncthreads();
    const int row0 = blockIdx.x * 16 + wave_id() * kRowsPerWave;
    const int valid = rows - row0;
    if (valid <= 0) return;
    const int lane = lane_id();
    const int g = lane / kLanesPerRow;
    const int q = lane % kLanesPerRow;
    const bool ok = g < valid;
    const int r = ok ? row0 + g : row0;
    const uint32_t* wrow = reinterpret_cast<const uint32_t*>(w + (size_t)r * K);
    float acc[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.0f;
    const int nblocks = K / 32;
    for (int b0 = 0; b0 < nblocks; b0 += 32) {
        const int nb = min(32, nblocks - b0);
        RowShare<32> rs;
        row_issue(rs, wrow + b0 * 16, nb, q);
        row_chains_acc<NT, 32>(rs, nb, xs + b0 * 32, K, q, acc);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float d = tree32_reduce(acc[t][0], acc[t][1]);
        if (q == 0 && ok) {
            d = tree32_finish(d, w + (size_t)r * K, xs + t * K, K);
            out[(size_t)t * rows + r] = to_bf16(d);
        }
    }
}

// out[t][r] = bf16(fold(W[r,:], x[t,:])): one thread per (row, token).
__global__ void k_linear_fold(const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
                              int rows, int K, int T, uint16_t* __restrict__ out) {
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < T * K; i += blockDim.x) xs[i] = from_bf16(x[i]);
    __syncthreads();
    int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    for (int t = 0; t < T; ++t) out[(size_t)t * rows + r] = to_bf16(fold_row(w + (size_t)r * K, xs + t * K, K));
}

__global__ void k_swiglu(const uint16_t* gate, const uint16_t* up, size_t n, uint16_t* out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = swiglu_bf16(gate[i], up[i], c_exp2_table);
}

__global__ void k_sigmoid(const uint16_t* in, size_t n, uint16_t* out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = sigmoid_bf16(in[i], c_exp2_table);
}

// dst = src, 16 bytes per thread and iteration (a grid-stride streaming copy).
__global__ void __launch_bounds__(256) k_copy_bytes(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                    size_t n16) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

__global__ void k_expf(const float* in, float* out, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = expf_glibc(in[i], c_exp2_table);
}

__global__ void k_scale_bf16(const uint16_t* in, uint16_t weight, size_t n, uint16_t* out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = to_bf16(mul_rn(from_bf16(in[i]), from_bf16(weight)));
}

// Top-k (and optionally scores) of T rows of `count` logits: one wave per row.
// With scores: max, exp(v - max), sequential sum, renormalised selection
// (src/router.rs:248-262). reject_nan: src/decoder_layer.rs:279-281.
__global__ void __launch_bounds__(64) k_select(const uint16_t* __restrict__ logits, int count,
                                               int k, int32_t* __restrict__ ids,
                                               uint16_t* __restrict__ scores, int reject_nan,
                                               int32_t* __restrict__ error) {
    __shared__ float ex[kMaxExperts];
    __shared__ int32_t sid[kMaxTopK];
    const uint16_t* lt = logits + (size_t)blockIdx.x * count;
    const int lane = lane_id();
    if (reject_nan) {
        int nan = 0;
        for (int e = lane; e < count; e += kWave) nan |= ((lt[e] & 0x7fffu) > 0x7f80u);
        if (__any(nan)) {
            // rejected: the token's ids read -1 (device callers see it there)
            if (lane == 0) atomicExch(error, 2);
            if (lane < k) ids[(size_t)blockIdx.x * k + lane] = -1;
            return;
        }
    }
    wave_topk<kMaxExperts / kWave>(lt, count, k, sid);
    __syncthreads();
    if (lane < k) ids[(size_t)blockIdx.x * k + lane] = sid[lane];
    if (scores == nullptr) return;
    float mx = -__builtin_inff();
    for (int e = lane; e < count; e += kWave) mx = fmaxf(mx, from_bf16(lt[e]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    for (int e = lane; e < count; e += kWave) ex[e] = expf_glibc(add_rn(from_bf16(lt[e]), -mx), c_exp2_table);
    __syncthreads();
    if (lane == 0) {
        float den = -0.0f;
        for (int e = 0; e < count; ++e) den = add_rn(den, ex[e]);
        float sel = -0.0f;
        for (int r = 0; r < k; ++r) sel = add_rn(sel, ex[sid[r]] / den);
        for (int r = 0; r < k; ++r) scores[(size_t)blockIdx.x * k + r] = to_bf16((ex[sid[r]] / den) / sel);
    }
}

// Ordered bf16 mixture of n weighted rows: mix = 0; for i: mix = bf16(mix + w_i)
// (src/expert.rs:953-955).
__global__ void k_mixture(const uint16_t* __restrict__ weighted, int n, int H,
                          uint16_t* __restrict__ out) {
    int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= H) return;
    uint32_t mix = to_bf16(0.0f);
    for (int i = 0; i < n; ++i) mix = add_bf16(mix, weighted[(size_t)i * H + h]);
    out[h] = (uint16_t)mix;
}

// Synthetic weights: dst[i] = table[u16(stream, first + i)] (fw_synth.h).
__global__ void k_generate(uint16_t* __restrict__ dst, size_t count, uint64_t stream,
                           uint64_t first, const uint16_t* __restrict__ table) {
    size_t quad = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t i0 = quad * 4;
    if (i0 >= count) return;
    // first is a multiple of 4, so one hash serves four elements
    uint64_t h = fw_mix64(stream + ((first + i0) >> 2));
    uint16_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = table[(uint32_t)(h >> (16 * j)) & 0xffffu];
    if (i0 + 4 <= count) {
        uint2 packed;
        packed.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
        packed.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
        *reinterpret_cast<uint2*>(dst + i0) = packed;
    } else {
        for (size_t j = 0; i0 + j < count; ++j) dst[i0 + j] = v[j];
    }
}

// Router bias column: router[e][H-1] = bias[e].
__global__ void k_router_bias(uint16_t* router, int E, int H, const uint16_t* bias) {
    int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < E) router[(size_t)e * H + H - 1] = bias[e];
}

}  // namespace fw

// ---- launch helpers ---------------------------------------------------------------------

namespace {

bool shape_ok_for_linear(size_t rows, size_t columns, std::string* why) {
    if (rows == 0 || columns == 0) {
        *why = "linear: rows and columns must be nonzero";
        return false;
    }
    if (rows > (1u << 30) || columns > 16384) {
        *why = "linear: rows must be < 2^30 and columns <= 16384";
        return false;
    }
    return true;
}

void launch_linear(const uint16_t* w, const uint16_t* x, int rows, int K, int T, uint16_t* out,
                   hipStream_t s) {
    dim3 grid((rows + 15) / 16);
    size_t shmem = (size_t)T * K * sizeof(float);
    // columns that are not a multiple of 32 still work (tail by one lane), but
    // the 16-lane sweep needs 4-byte aligned rows, so K must be even there.
    switch (T) {
        case 1: hipLaunchKernelGGL(k_linear_tree32<1>, grid, dim3(256), shmem, s, w, x, rows, K, out); break;
        case 2: hipLaunchKernelGGL(k_linear_tree32<2>, grid, dim3(256), shmem, s, w, x, rows, K, out); break;
        case 3: hipLaunchKernelGGL(k_linear_tree32<3>, grid, dim3(256), shmem, s, w, x, rows, K, out); break;
        default: hipLaunchKernelGGL(k_linear_tree32<4>, grid, dim3(256), shmem, s, w, x, rows, K, out); break;
    }
    check(hipGetLastError(), "k_linear_tree32 launch");
}

}  // namespace

// ---- resident context ---------------------------------------------------------------------

struct firewing_hip_context {
    firewing_hip_shape shape{};
    int device = 0;
    char device_name[256] = {0};
    int cu_count = 0;
    uint64_t wall_clock_hz = 100000000ULL;
    hipStream_t stream = nullptr;
    // the context's last queued work, on whichever stream it ran: every call
    // waits for it and then records its own (calls share the scratch below)
    hipEvent_t last = nullptr;
    // resident banks
    std::vector<uint16_t*> router;  // [E + 1][H] per layer
    std::vector<uint16_t*> gate_up, down, shared_gate, shared_up, shared_down;
    DecodeLayer* d_layers = nullptr;  // [L]
    // interleaved token chains: for each chain count c = 2..kMaxTokens, [L * c]
    // entries, entry v = layer v / c (see vlayers_offset)
    DecodeLayer* d_vlayers = nullptr;
    uint16_t* d_weight_table = nullptr;
    // decode scratch sized for L layers and T <= 4
    uint16_t* xin = nullptr;     // [T][H] host input staged for the launch
    uint16_t* xfinal = nullptr;  // [T][H] residual after the last layer
    uint16_t *out = nullptr, *scores = nullptr, *sig = nullptr;
    int32_t* ids = nullptr;
    uint64_t *xw = nullptr, *logits = nullptr, *shared_act = nullptr, *act = nullptr;  // tagged words
    uint32_t* counters = nullptr;
    uint32_t* flags = nullptr;  // phase flags (epoch of the completed phase)
    int32_t* error = nullptr;
    uint32_t epoch = 0;  // tag of the last launch
    int grid[kMaxTokens + 1] = {0};
    uint64_t* trace = nullptr;  // profiling builds: per-task timestamps of the next launch
    DecodeParams* d_params = nullptr;  // device copy of the last launch's parameters
    DecodeParams last_params{};
    bool params_valid = false;
    double timeout_seconds = 10.0;  // per dependency wait (FIREWING_WAIT_TIMEOUT_S)
    // many-token (prefill) scratch, grown to the largest token count seen
    struct Prefill {
        size_t tokens = 0;  // capacity
        uint16_t *x = nullptr, *out = nullptr, *mixture = nullptr, *logits = nullptr, *gate = nullptr;
        uint16_t *scores = nullptr, *act = nullptr, *weighted = nullptr;
        uint16_t* silu = nullptr;  // the SiLU table (built once)
        int32_t* ids = nullptr;
        int32_t* redo = nullptr;   // [token tiles][row tiles] of k_pf_router_mx
        PfGroups g{};
        std::vector<void*> owned;
    } pf;
    // mlp hyper-connection per layer (installed on demand) and its scratch for T <= 4
    struct Hyper {
        int streams = 0, lowrank = 0;
        std::vector<uint16_t*> norm, down, up, inject;  // [S*H], [R][S*H], [S*H][R], [S][S*H]
        std::vector<void*> owned;
        uint16_t *normed = nullptr, *mix_down = nullptr, *scaled = nullptr, *silu = nullptr, *mix_up = nullptr;
        uint16_t *input_mix = nullptr, *products = nullptr, *mixed = nullptr, *inject_out = nullptr;
        uint16_t *inject_scaled = nullptr, *inject_sigmoid = nullptr, *weights = nullptr;
        uint16_t *post = nullptr, *layer_out = nullptr, *inj_products = nullptr;
    } hc;
    // LM head [vocab][H] (installed on demand) and its scratch for T <= 4
    struct LmHead {
        size_t vocab = 0;
        uint16_t* weight = nullptr;   // + kLineSharePad bytes
        uint16_t* logits = nullptr;   // [T][vocab]
        uint16_t* cand_key = nullptr;  // [T][chunks][k]: the chunks' top keys (total-order bf16 keys)
        uint16_t* cand_pos = nullptr;  // [T][chunks][k]: and their positions in the chunk
        int32_t* ids = nullptr;       // [T][kMaxLmTopK]
        uint16_t* values = nullptr;   // [T][kMaxLmTopK]
        int grid = 0;                 // workgroups of k_lm_head
    } lm;
};

namespace {

template <typename T>
T* dalloc(size_t count) {
    void* p = nullptr;
    check(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)), "hipMalloc");
    return static_cast<T*>(p);
}

// A call's work on stream s runs after every earlier call on the context
// (whatever stream that used) and becomes the context's last work: the
// constructor makes s wait for the last recorded work, the destructor records
// s's queue end (also when the call fails part-way, so nothing queued is left
// unordered).
struct Ordered {
    firewing_hip_context* c;
    hipStream_t s;
    Ordered(firewing_hip_context* ctx, void* stream)
        : c(ctx), s(stream ? static_cast<hipStream_t>(stream) : ctx->stream) {
        check(hipStreamWaitEvent(s, c->last, 0), "hipStreamWaitEvent");
    }
    ~Ordered() { (void)hipEventRecord(c->last, s); }
    Ordered(const Ordered&) = delete;
    Ordered& operator=(const Ordered&) = delete;
};

bool validate_shape(const firewing_hip_shape& s, std::string* why) {
    auto bad = [&](const char* m) {
        *why = m;
        return false;
    };
    if (s.hidden == 0 || s.hidden % 32 || s.hidden > (size_t)kMaxHidden)
        return bad("hidden must be a nonzero multiple of 32 and <= 2560");
    if (s.intermediate == 0 || s.intermediate % 32 || s.intermediate > 1024)
        return bad("intermediate must be a nonzero multiple of 32 and <= 1024");
    if (s.shared_intermediate == 0 || s.shared_intermediate % 32 || s.shared_intermediate > 1024)
        return bad("shared_intermediate must be a nonzero multiple of 32 and <= 1024");
    if (s.experts == 0 || s.experts > (size_t)kMaxExperts) return bad("experts must be in [1, 1024]");
    if (s.top_k == 0 || s.top_k > (size_t)kMaxTopK || s.top_k > s.experts)
        return bad("top_k must be in [1, min(32, experts)]");
    if (s.layers == 0 || s.layers > 4096) return bad("layers must be in [1, 4096]");
    return true;
}

// Kernel variant for T tokens and the context's shape: hidden rows of up to
// 64 blocks (H <= 2048) or 80 (H <= 2560); down rows of up to 16 blocks
// (I, Is <= 512), 20 (<= 640, one token: the fused C task) or 32 (<= 1024);
// top-k over up to 512 experts or 1024.
const void* decode_kernel(const firewing_hip_context* c, int T) {
    const bool wide_h = c->shape.hidden > 2048;
    const size_t max_i = std::max(c->shape.intermediate, c->shape.shared_intermediate);
    const bool wide_i = max_i > 512;
    const bool wide_e = c->shape.experts > 512;
    if (T == 1 && wide_i && max_i <= 640) {
        if (wide_e) return wide_h ? reinterpret_cast<const void*>(&k_moe_decode<1, 80, 20, 16>)
                                  : reinterpret_cast<const void*>(&k_moe_decode<1, 64, 20, 16>);
        return wide_h ? reinterpret_cast<const void*>(&k_moe_decode<1, 80, 20, 8>)
                      : reinterpret_cast<const void*>(&k_moe_decode<1, 64, 20, 8>);
    }
#define FW_DECODE_VARIANT(NT, TK)                                                                      \
    if (T == NT && wide_e == (TK == 16)) {                                                             \
        if (!wide_h && !wide_i) return reinterpret_cast<const void*>(&k_moe_decode<NT, 64, 16, TK>); \
        if (!wide_h && wide_i) return reinterpret_cast<const void*>(&k_moe_decode<NT, 64, 32, TK>);  \
        if (wide_h && !wide_i) return reinterpret_cast<const void*>(&k_moe_decode<NT, 80, 16, TK>);  \
        return reinterpret_cast<const void*>(&k_moe_decode<NT, 80, 32, TK>);                         \
    }
    FW_DECODE_VARIANT(1, 8)
    FW_DECODE_VARIANT(2, 8)
    FW_DECODE_VARIANT(3, 8)
    FW_DECODE_VARIANT(4, 8)
    FW_DECODE_VARIANT(1, 16)
    FW_DECODE_VARIANT(2, 16)
    FW_DECODE_VARIANT(3, 16)
    FW_DECODE_VARIANT(4, 16)
#undef FW_DECODE_VARIANT
    throw HipError{"no decode kernel for this token count"};
}

int decode_grid(const firewing_hip_context* c, int T) {
    int per_cu = 0;
    check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel(c, T), 256, 0),
          "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (per_cu < 1) throw HipError{"decode kernel cannot be resident"};
    return per_cu * c->cu_count;
}

// First entry of the interleaved layer table for `chains` chains (2..kMaxTokens)
// over L layers: the tables for 2, 3, ... chains follow one another.
size_t vlayers_offset(size_t L, int chains) { return L * (size_t)((chains - 2) * (chains + 1) / 2); }

// How one-token work runs at this shape. The fused C task (the one-token
// kernel variants with down rows of up to 640 columns, at most 11 staged
// activation vectors) either carries two gate/up pairs itself (kFusedPairs:
// every C task of a layer resident at once, one combine workgroup each; the
// B tasks past the rows role's one per workgroup coming to exactly two pairs
// per C task; I, Is multiples of 256 and H of 512 for its row copies) or
// none (kFusedNoPairs: the rows role runs every B task; combine workgroups may
// take several C tasks per layer). kUnfused: the multi-token kernel.
enum OneTokenMode { kUnfused = 0, kFusedNoPairs = 1, kFusedPairs = 2 };

OneTokenMode one_token_mode(const firewing_hip_context* c) {
    const firewing_hip_shape& sh = c->shape;
    const size_t max_i = std::max(sh.intermediate, sh.shared_intermediate);
    const int mbh = sh.hidden > 2048 ? 80 : 64;
    const int mbi = max_i <= 512 ? 16 : (max_i <= 640 ? 20 : 32);
    if (!fused_combine(1, mbh, mbi) || sh.top_k + 1 > (size_t)kDirectVectors) return kUnfused;
    const int n_c = (int)(sh.hidden / kRowsPerCTask);
    const int n_b = (int)(sh.top_k * (sh.intermediate / kPairsPerTask));
    const int grid = c->grid[1];
    const int g_comb = std::min(n_c, grid / 2);
    const int nb_rows = std::min(n_b, grid - g_comb);
    const bool pairs = g_comb == n_c && sh.intermediate % 256 == 0 && sh.shared_intermediate % 256 == 0 &&
                       sh.hidden % 512 == 0 &&
                       (long)n_b * kPairsPerTask - (long)nb_rows * kPairsPerTask == 2L * n_c;
    return pairs ? kFusedPairs : kFusedNoPairs;
}

bool one_token_fused(const firewing_hip_context* c) { return one_token_mode(c) != kUnfused; }

// Launch the persistent kernel over layers [first, first + n) for T tokens.
// x_in holds the input of the first layer ([T][H] bf16, 4-byte aligned).
// Where one-token work runs fused, T >= 2 tokens run as T independent
// one-token chains interleaved by layer (launch layer l * T + t = layer l of
// token t; the outputs' [layer][token] order is the same), so the chains'
// serial steps overlap; otherwise the T-token kernel reads each union expert
// once for all its tokens.
void launch_decode(firewing_hip_context* c, size_t first, size_t n, int T, int order,
                   bool prenorm, bool bias_feature, const uint16_t* x_in, uint16_t* x_final,
                   hipStream_t s) {
    const firewing_hip_shape& sh = c->shape;
    const OneTokenMode mode = one_token_mode(c);
    const bool fused = mode != kUnfused;
    const int chains = (T >= 2 && fused) ? T : 1;
    DecodeParams p{};
    p.layers = c->d_layers + first;
    if (chains > 1) {
        T = 1;
        p.layers = c->d_vlayers + vlayers_offset(c->shape.layers, chains) + first * chains;
        n *= chains;
    }
    p.nlayers = (int)n;
    p.chains = chains;
    p.T = T;
    p.H = (int)sh.hidden;
    p.I = (int)sh.intermediate;
    p.E = (int)sh.experts;
    p.K = (int)sh.top_k;
    p.Is = (int)sh.shared_intermediate;
    p.order = order;
    p.prenorm = prenorm ? 1 : 0;
    p.bias_feature = bias_feature ? 1 : 0;
    p.S = p.K * T;
    const size_t H = sh.hidden, E = sh.experts;
    const size_t S = (size_t)p.S, I = sh.intermediate, Is = sh.shared_intermediate;
    p.x_in = x_in;
    p.xw = c->xw;
    p.logits = c->logits;
    p.ls = logit_stride((int)E);
    p.gi = p.ls - 2;
    p.shared_act = c->shared_act;
    p.act = c->act;
    p.x_final = x_final;
    p.out = c->out;
    p.ids = c->ids;
    p.scores = c->scores;
    p.sig = c->sig;
    p.counters = c->counters;
    p.flags = c->flags;
    p.error = c->error;
    p.limit_ticks = (uint64_t)(c->timeout_seconds * (double)c->wall_clock_hz);
    p.n_router = (int)((E + kRouterRowsPerTask - 1) / kRouterRowsPerTask) + 1;
    p.n_shared = (int)((Is + kPairsPerTask - 1) / kPairsPerTask);
    p.n_b = (int)(S * (I / kPairsPerTask));
    p.n_c = (int)(H / kRowsPerCTask);
    // Roles: the combine role gets one workgroup per C task of a layer where
    // the grid allows (so every task's down rows are in flight before the
    // gate/up phase ends), at most half of the grid. The rows role takes one
    // B task per workgroup and layer (the kernels for two or more tokens: as
    // many as even out the two roles' lists). B tasks beyond that: with one token, when
    // they come to two gate/up pairs per C task, wave 0 of each C task computes
    // them (the one-token kernel, which requires this: every C task of a layer
    // is resident at once and publishes its pairs before waiting for the
    // phase); otherwise they go to the combine role ahead of its C tasks (the
    // kernels for two or more tokens, which also run one-token steps that
    // cannot be fused).
    auto roles = [&](int kt) {
        const int grid = c->grid[kt];
        p.g_comb = std::min(p.n_c, grid / 2);
        p.g_rows = grid - p.g_comb;
        p.nb_rows = std::min(p.n_b, p.g_rows);
        if (kt >= 2) {
            // several B tasks per rows workgroup: even out the two roles'
            // task lists, a C task counted as two B tasks (the B tasks left to
            // the combine role are the last union slots, often empty)
            const int even = (p.n_b + 2 * p.n_c - p.n_router - p.n_shared) / 2;
            p.nb_rows = std::min(p.n_b, std::max(p.nb_rows, even));
        }
        if (p.g_comb < 1 || p.g_rows < 1) throw HipError{"decode grid too small for its roles"};
    };
    int kt = T;  // token count of the kernel variant
    p.cpairs = 0;
    if (T == 1) {
        roles(1);
        if (!fused) {
            kt = 2;
        } else if (chains == 1 && mode == kFusedPairs) {
            p.cpairs = 2;
        } else {
            // no pairs on the C tasks: with interleaved chains a combine
            // workgroup runs the chains' C tasks one after another (pairs
            // there would lengthen every chain), and without the exact split
            // there are none to carry; the rows role runs every B task
            p.nb_rows = p.n_b;
        }
    }
    if (kt != 1) roles(kt);
    p.n_gu = p.n_shared + (p.cpairs > 0 ? p.nb_rows + p.n_c : p.n_b);
    p.cu_count = c->cu_count;
    // the fused one-token C task reads its activations by their tags and
    // rank-ordered slots
    p.input_by_tags = kt == 1 ? 1 : 0;
    p.rank_slots = kt == 1 ? 1 : 0;
    p.trace = c->trace;
    // The kernel reads its parameters from a device copy; upload only on change
    // (the copy is stream-ordered before the launch; pageable source, staged).
    if (std::memcmp(&p, &c->last_params, sizeof p) != 0 || !c->params_valid) {
        c->last_params = p;
        c->params_valid = true;
        check(hipMemcpyAsync(c->d_params, &c->last_params, sizeof p, hipMemcpyHostToDevice, s),
              "upload decode params");
    }
    const DecodeParams* dp = c->d_params;
    // a fresh tag for this launch's exchanged words (0 is never used)
    c->epoch = c->epoch + 1 == 0 ? 1 : c->epoch + 1;
    uint32_t epoch = c->epoch;
    void* args[] = {&dp, &epoch};
    const void* fn = decode_kernel(c, kt);
    check(hipLaunchCooperativeKernel(fn, dim3(c->grid[kt]), dim3(256), args, 0, s),
          "hipLaunchCooperativeKernel(k_moe_decode)");
}

bool check_device_error(firewing_hip_context* c, hipStream_t s) {
    int32_t err = 0;
    check(hipMemcpyAsync(&err, c->error, sizeof err, hipMemcpyDeviceToHost, s), "hipMemcpyAsync error word");
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (err != 0) {
        int32_t zero = 0;
        check(hipMemcpy(c->error, &zero, sizeof zero, hipMemcpyHostToDevice), "reset error word");
        if (err == 2) return fail("router produced a NaN logit (rejected, src/decoder_layer.rs:279-281)");
        return fail("persistent decode kernel: a dependency wait exceeded its time limit");
    }
    return true;
}

}  // namespace

// ---- scratch of the entry point that allocates nothing ----------------------------------
//
// firewing_hip_route_bf16_noalloc keeps its intermediate logits (when the caller
// takes none) and the top-k kernel's NaN word here instead of in memory it
// allocates. One copy per GPU, held until the process ends; in host code the
// array's name is only a handle: its device address comes from
// hipGetSymbolAddress, once per device.
constexpr size_t kRouteScratchHeader = 256;               // the NaN word, then padding
constexpr size_t kRouteScratchLogitBytes = (size_t)1 << 20;  // logits: tokens * experts * 2 bytes
static __device__ __align__(256) uint8_t scratch[kRouteScratchHeader + kRouteScratchLogitBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxScratchDevices] = {};

// Device address of `scratch` on `device` (the current device).
void* route_scratch(int device) {
    if (device < 0 || device >= kMaxScratchDevices) throw HipError{"route_bf16_noalloc: device index out of range"};
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_address[device] == nullptr) {
        void* p = nullptr;
        check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (p == nullptr) throw HipError{"hipGetSymbolAddress(scratch) returned null"};
        g_scratch_address[device] = p;
    }
    return g_scratch_address[device];
}

}  // namespace

// ---- C ABI ------------------------------------------------------------------------------

extern "C" {

const char* firewing_hip_last_error(void) { return g_last_error.c_str(); }

void firewing_hip_synth_hidden(uint64_t seed, uint32_t first_token, uint32_t tokens,
                               uint32_t hidden, bool bias_feature, uint16_t* out) {
    static std::vector<uint16_t> unit_table;
    if (unit_table.empty()) {
        std::vector<uint16_t> table(65536);
        fw_synth_normal_table(1.0, table.data());
        unit_table.swap(table);
    }
    fw_synth_hidden(seed, first_token, tokens, hidden, bias_feature ? 1 : 0, unit_table.data(), out);
}

void firewing_hip_expf_host(const float* in, float* out, size_t count) {
    for (size_t i = 0; i < count; ++i) out[i] = expf_glibc(in[i], kExp2TableHost);
}

bool firewing_hip_expf_device(const float* in, float* out, size_t count) {
    return guarded([&] {
        if (!in || !out) return fail("expf_device: null pointer");
        DeviceBuffer din(count * 4), dout(count * 4);
        upload(din.ptr, in, count * 4, nullptr);
        if (count) {
            hipLaunchKernelGGL(k_expf, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, nullptr,
                               din.as<float>(), dout.as<float>(), count);
            check(hipGetLastError(), "k_expf launch");
        }
        download(out, dout.ptr, count * 4, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_copy_bytes(void* dst, const void* src, size_t bytes, void* stream) {
    return guarded([&] {
        if (!dst || !src) return fail("copy_bytes: null pointer");
        if (bytes % 16) return fail("copy_bytes: bytes must be a multiple of 16");
        if (bytes == 0) return true;
        const size_t n16 = bytes / 16;
        const unsigned grid = (unsigned)std::min<size_t>((n16 + 255) / 256, 4096);
        hipLaunchKernelGGL(k_copy_bytes, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<uint4*>(dst), static_cast<const uint4*>(src), n16);
        check(hipGetLastError(), "k_copy_bytes launch");
        return true;
    });
}

bool firewing_hip_linear_bf16(const uint16_t* weight, const uint16_t* input, size_t rows,
                              size_t columns, uint16_t* out) {
    return guarded([&] {
        if (!weight || !input || !out) return fail("linear_bf16: null pointer");
        std::string why;
        if (!shape_ok_for_linear(rows, columns, &why)) return fail(why);
        if (columns % 2) return fail("linear_bf16: columns must be even");
        DeviceBuffer dw(rows * columns * 2), dx(columns * 2), dout(rows * 2);
        upload(dw.ptr, weight, rows * columns * 2, nullptr);
        upload(dx.ptr, input, columns * 2, nullptr);
        launch_linear(dw.as<uint16_t>(), dx.as<uint16_t>(), (int)rows, (int)columns, 1,
                      dout.as<uint16_t>(), nullptr);
        download(out, dout.ptr, rows * 2, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_swiglu_bf16(const uint16_t* gate, const uint16_t* up, size_t count,
                              uint16_t* out) {
    return guarded([&] {
        if (!gate || !up || !out) return fail("swiglu_bf16: null pointer");
        if (count == 0) return true;
        DeviceBuffer dg(count * 2), du(count * 2), dout(count * 2);
        upload(dg.ptr, gate, count * 2, nullptr);
        upload(du.ptr, up, count * 2, nullptr);
        hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, nullptr,
                           dg.as<uint16_t>(), du.as<uint16_t>(), count, dout.as<uint16_t>());
        check(hipGetLastError(), "k_swiglu launch");
        download(out, dout.ptr, count * 2, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_sigmoid_bf16(const uint16_t* input, size_t count, uint16_t* out) {
    return guarded([&] {
        if (!input || !out) return fail("sigmoid_bf16: null pointer");
        if (count == 0) return true;
        DeviceBuffer din(count * 2), dout(count * 2);
        upload(din.ptr, input, count * 2, nullptr);
        hipLaunchKernelGGL(k_sigmoid, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, nullptr,
                           din.as<uint16_t>(), count, dout.as<uint16_t>());
        check(hipGetLastError(), "k_sigmoid launch");
        download(out, dout.ptr, count * 2, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_topk_bf16(const uint16_t* values, size_t count, size_t k, size_t* indices) {
    return guarded([&] {
        if (!values || !indices || k == 0 || k > count) return fail("invalid top-k request");
        if (count > (size_t)kMaxExperts || k > (size_t)kMaxTopK)
            return fail("top-k: count must be <= 1024 and k <= 32");
        DeviceBuffer dv(count * 2), dids(k * 4), derr(4);
        upload(dv.ptr, values, count * 2, nullptr);
        check(hipMemsetAsync(derr.ptr, 0, 4, nullptr), "hipMemsetAsync");
        hipLaunchKernelGGL(k_select, dim3(1), dim3(64), 0, nullptr, dv.as<uint16_t>(), (int)count,
                           (int)k, dids.as<int32_t>(), (uint16_t*)nullptr, 0, derr.as<int32_t>());
        check(hipGetLastError(), "k_select launch");
        std::vector<int32_t> ids(k);
        download(ids.data(), dids.ptr, k * 4, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        for (size_t i = 0; i < k; ++i) indices[i] = (size_t)ids[i];
        return true;
    });
}

bool firewing_hip_route_bf16(const uint16_t* weight, const uint16_t* hidden, size_t tokens,
                             size_t experts, size_t width, size_t top_k, int order,
                             size_t* ids, uint16_t* scores, uint16_t* logits) {
    return guarded([&] {
        if (!weight || !hidden || !ids || !scores) return fail("route_bf16: null pointer");
        if (tokens == 0 || tokens > 4096) return fail("route_bf16: tokens must be in [1, 4096]");
        if (experts == 0 || experts > (size_t)kMaxExperts) return fail("route_bf16: experts must be in [1, 1024]");
        if (top_k == 0 || top_k > experts || top_k > (size_t)kMaxTopK)
            return fail("route_bf16: top_k must be in [1, min(32, experts)]");
        if (order != FIREWING_HIP_LOGITS_TREE32 && order != FIREWING_HIP_LOGITS_FOLD)
            return fail("route_bf16: unknown logit order");
        std::string why;
        if (!shape_ok_for_linear(experts, width, &why)) return fail(why);
        if (width % 2) return fail("route_bf16: width must be even");
        DeviceBuffer dw(experts * width * 2), dx(tokens * width * 2), dl(tokens * experts * 2);
        DeviceBuffer dids(tokens * top_k * 4), dsc(tokens * top_k * 2), derr(4);
        upload(dw.ptr, weight, experts * width * 2, nullptr);
        upload(dx.ptr, hidden, tokens * width * 2, nullptr);
        check(hipMemsetAsync(derr.ptr, 0, 4, nullptr), "hipMemsetAsync");
        // up to 4 tokens per launch share each weight read; x stays <= 64 KiB of LDS
        const size_t per_launch = std::max<size_t>(1, std::min<size_t>(4, 16384 / width));
        if (order == FIREWING_HIP_LOGITS_TREE32) {
            for (size_t t0 = 0; t0 < tokens; t0 += per_launch) {
                int T = (int)std::min<size_t>(per_launch, tokens - t0);
                launch_linear(dw.as<uint16_t>(), dx.as<uint16_t>() + t0 * width, (int)experts,
                              (int)width, T, dl.as<uint16_t>() + t0 * experts, nullptr);
            }
        } else {
            for (size_t t0 = 0; t0 < tokens; t0 += per_launch) {
                int T = (int)std::min<size_t>(per_launch, tokens - t0);
                size_t shmem = (size_t)T * width * 4;
                hipLaunchKernelGGL(k_linear_fold, dim3((unsigned)((experts + 63) / 64)), dim3(64),
                                   shmem, nullptr, dw.as<uint16_t>(), dx.as<uint16_t>() + t0 * width,
                                   (int)experts, (int)width, T, dl.as<uint16_t>() + t0 * experts);
                check(hipGetLastError(), "k_linear_fold launch");
            }
        }
        // k_linear_* write token-major [T][rows]: already [tokens][experts]
        hipLaunchKernelGGL(k_select, dim3((unsigned)tokens), dim3(64), 0, nullptr,
                           dl.as<uint16_t>(), (int)experts, (int)top_k, dids.as<int32_t>(),
                           dsc.as<uint16_t>(), order == FIREWING_HIP_LOGITS_TREE32 ? 1 : 0,
                           derr.as<int32_t>());
        check(hipGetLastError(), "k_select launch");
        std::vector<int32_t> hid(tokens * top_k);
        int32_t err = 0;
        download(hid.data(), dids.ptr, hid.size() * 4, nullptr);
        download(scores, dsc.ptr, tokens * top_k * 2, nullptr);
        if (logits) download(logits, dl.ptr, tokens * experts * 2, nullptr);
        download(&err, derr.ptr, 4, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        if (err == 2) return fail("decoder-layer router received unsupported logits (NaN)");
        for (size_t i = 0; i < hid.size(); ++i) ids[i] = (size_t)hid[i];
        return true;
    });
}

bool firewing_hip_route_bf16_noalloc(const uint16_t* weight, const uint16_t* hidden, size_t tokens,
                                     size_t experts, size_t width, size_t top_k, int order, int32_t* ids,
                                     uint16_t* scores, uint16_t* logits, void* stream) {
    return guarded([&] {
        if (!weight || !hidden || !ids || !scores) return fail("route_bf16_noalloc: null pointer");
        if (tokens == 0 || tokens > 4096) return fail("route_bf16_noalloc: tokens must be in [1, 4096]");
        if (experts == 0 || experts > (size_t)kMaxExperts)
            return fail("route_bf16_noalloc: experts must be in [1, 1024]");
        if (top_k == 0 || top_k > experts || top_k > (size_t)kMaxTopK)
            return fail("route_bf16_noalloc: top_k must be in [1, min(32, experts)]");
        if (order != FIREWING_HIP_LOGITS_TREE32 && order != FIREWING_HIP_LOGITS_FOLD)
            return fail("route_bf16_noalloc: unknown logit order");
        std::string why;
        if (!shape_ok_for_linear(experts, width, &why)) return fail("route_bf16_noalloc: " + why);
        if (width % 2) return fail("route_bf16_noalloc: width must be even");
        if (reinterpret_cast<uintptr_t>(weight) % 4 || reinterpret_cast<uintptr_t>(hidden) % 2)
            return fail("route_bf16_noalloc: weight must be 4-byte aligned and hidden 2-byte aligned");
        if (!logits && tokens * experts * 2 > kRouteScratchLogitBytes)
            return fail("route_bf16_noalloc: without a logits output, tokens * experts must be <= 524288 "
                        "(the logits live in the library's 1 MiB scratch)");
        int device = 0;
        check(hipGetDevice(&device), "hipGetDevice");
        char* base = static_cast<char*>(route_scratch(device));
        int32_t* error = reinterpret_cast<int32_t*>(base);  // written on a NaN logit, read by no one
        uint16_t* lg = logits ? logits : reinterpret_cast<uint16_t*>(base + kRouteScratchHeader);
        hipStream_t s = static_cast<hipStream_t>(stream);
        const size_t per_launch = std::max<size_t>(1, std::min<size_t>(4, 16384 / width));
        for (size_t t0 = 0; t0 < tokens; t0 += per_launch) {
            const int T = (int)std::min<size_t>(per_launch, tokens - t0);
            if (order == FIREWING_HIP_LOGITS_TREE32) {
                launch_linear(weight, hidden + t0 * width, (int)experts, (int)width, T, lg + t0 * experts, s);
            } else {
                hipLaunchKernelGGL(k_linear_fold, dim3((unsigned)((experts + 63) / 64)), dim3(64),
                                   (size_t)T * width * 4, s, weight, hidden + t0 * width, (int)experts,
                                   (int)width, T, lg + t0 * experts);
                check(hipGetLastError(), "k_linear_fold launch");
            }
        }
        hipLaunchKernelGGL(k_select, dim3((unsigned)tokens), dim3(64), 0, s, lg, (int)experts, (int)top_k, ids,
                           scores, order == FIREWING_HIP_LOGITS_TREE32 ? 1 : 0, error);
        check(hipGetLastError(), "k_select launch");
        return true;
    });
}

bool firewing_hip_expert_bf16(const uint16_t* gate_up_weight, const uint16_t* down_weight,
                              const uint16_t* hidden, size_t hidden_size,
                              size_t intermediate, uint16_t route_weight,
                              uint16_t* gate_up, uint16_t* swiglu, uint16_t* down,
                              uint16_t* weighted) {
    return guarded([&] {
        if (!gate_up_weight || !down_weight || !hidden) return fail("expert_bf16: null pointer");
        std::string why;
        if (!shape_ok_for_linear(2 * intermediate, hidden_size, &why)) return fail(why);
        if (!shape_ok_for_linear(hidden_size, intermediate, &why)) return fail(why);
        if (hidden_size % 2 || intermediate % 2) return fail("expert_bf16: sizes must be even");
        const size_t H = hidden_size, I = intermediate;
        DeviceBuffer dgu(2 * I * H * 2), ddn(H * I * 2), dx(H * 2), dgo(2 * I * 2), dact(I * 2);
        DeviceBuffer ddo(H * 2), dwo(H * 2);
        upload(dgu.ptr, gate_up_weight, 2 * I * H * 2, nullptr);
        upload(ddn.ptr, down_weight, H * I * 2, nullptr);
        upload(dx.ptr, hidden, H * 2, nullptr);
        launch_linear(dgu.as<uint16_t>(), dx.as<uint16_t>(), (int)(2 * I), (int)H, 1,
                      dgo.as<uint16_t>(), nullptr);
        hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((I + 255) / 256)), dim3(256), 0, nullptr,
                           dgo.as<uint16_t>(), dgo.as<uint16_t>() + I, I, dact.as<uint16_t>());
        check(hipGetLastError(), "k_swiglu launch");
        launch_linear(ddn.as<uint16_t>(), dact.as<uint16_t>(), (int)H, (int)I, 1,
                      ddo.as<uint16_t>(), nullptr);
        hipLaunchKernelGGL(k_scale_bf16, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, nullptr,
                           ddo.as<uint16_t>(), route_weight, H, dwo.as<uint16_t>());
        check(hipGetLastError(), "k_scale_bf16 launch");
        if (gate_up) download(gate_up, dgo.ptr, 2 * I * 2, nullptr);
        if (swiglu) download(swiglu, dact.ptr, I * 2, nullptr);
        if (down) download(down, ddo.ptr, H * 2, nullptr);
        if (weighted) download(weighted, dwo.ptr, H * 2, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_create(const firewing_hip_shape* shape, firewing_hip_context** out) {
    if (out) *out = nullptr;
    firewing_hip_context* c = nullptr;
    bool ok = guarded([&] {
        if (!shape || !out) return fail("create: null pointer");
        std::string why;
        if (!validate_shape(*shape, &why)) return fail(why);
        c = new firewing_hip_context();
        c->shape = *shape;
        check(hipGetDevice(&c->device), "hipGetDevice");
        hipDeviceProp_t prop;
        check(hipGetDeviceProperties(&prop, c->device), "hipGetDeviceProperties");
        std::snprintf(c->device_name, sizeof c->device_name, "%s (%s)", prop.name, prop.gcnArchName);
        c->cu_count = prop.multiProcessorCount;
        int wall_khz = 0;
        if (hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, c->device) == hipSuccess &&
            wall_khz >= 1000 && wall_khz <= 10000000)
            c->wall_clock_hz = (uint64_t)wall_khz * 1000ULL;
        if (!prop.cooperativeLaunch) return fail("device does not support cooperative launch");
        if (const char* env = std::getenv("FIREWING_WAIT_TIMEOUT_S")) {
            double v = std::atof(env);
            if (v > 0.0 && v <= 600.0) c->timeout_seconds = v;
        }
        check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
        check(hipEventCreateWithFlags(&c->last, hipEventDisableTiming), "hipEventCreate");
        const size_t L = shape->layers, H = shape->hidden, I = shape->intermediate;
        const size_t E = shape->experts, Is = shape->shared_intermediate, K = shape->top_k;
        c->router.assign(L, nullptr);
        c->gate_up.assign(L, nullptr);
        c->down.assign(L, nullptr);
        c->shared_gate.assign(L, nullptr);
        c->shared_up.assign(L, nullptr);
        c->shared_down.assign(L, nullptr);
        std::vector<DecodeLayer> layers(L);
        for (size_t l = 0; l < L; ++l) {
            c->router[l] = dalloc<uint16_t>((E + 1) * H + kLineSharePad / 2);
            c->gate_up[l] = dalloc<uint16_t>(E * 2 * I * H + kLineSharePad / 2);
            c->down[l] = dalloc<uint16_t>(E * H * I + kLineSharePad / 2);
            // gate and up rows of the shared expert in one allocation (the
            // decode kernel addresses both from shared_gate)
            c->shared_gate[l] = dalloc<uint16_t>(2 * Is * H + kLineSharePad / 2);
            c->shared_up[l] = c->shared_gate[l] + Is * H;
            c->shared_down[l] = dalloc<uint16_t>(H * Is + kLineSharePad / 2);
            layers[l] = DecodeLayer{c->router[l], c->gate_up[l], c->down[l], c->shared_gate[l],
                                    c->shared_up[l], c->shared_down[l]};
        }
        c->d_layers = dalloc<DecodeLayer>(L);
        check(hipMemcpy(c->d_layers, layers.data(), L * sizeof(DecodeLayer), hipMemcpyHostToDevice),
              "hipMemcpy layers");
        std::vector<DecodeLayer> vlayers(vlayers_offset(L, kMaxTokens + 1));
        for (int chains = 2; chains <= kMaxTokens; ++chains)
            for (size_t v = 0; v < L * chains; ++v) vlayers[vlayers_offset(L, chains) + v] = layers[v / chains];
        c->d_vlayers = dalloc<DecodeLayer>(vlayers.size());
        check(hipMemcpy(c->d_vlayers, vlayers.data(), vlayers.size() * sizeof(DecodeLayer), hipMemcpyHostToDevice),
              "hipMemcpy interleaved layers");
        const size_t T = kMaxTokens, S = K * T;
        c->xin = dalloc<uint16_t>(T * H);
        c->xfinal = dalloc<uint16_t>(T * H);
        c->out = dalloc<uint16_t>(L * T * H);
        c->ids = dalloc<int32_t>(L * T * K);
        c->scores = dalloc<uint16_t>(L * T * K);
        c->sig = dalloc<uint16_t>(L * T);
        c->xw = dalloc<uint64_t>((L + 1) * T * H / 2);
        c->logits = dalloc<uint64_t>(L * T * logit_stride((int)E) / 2);
        c->shared_act = dalloc<uint64_t>(L * T * Is / 2);
        c->act = dalloc<uint64_t>(L * S * T * I / 2);
        // tags start at zero: no launch uses epoch 0
        check(hipMemset(c->xw, 0, (L + 1) * T * H / 2 * 8), "hipMemset");
        check(hipMemset(c->logits, 0, L * T * logit_stride((int)E) / 2 * 8), "hipMemset");
        check(hipMemset(c->shared_act, 0, L * T * Is / 2 * 8), "hipMemset");
        check(hipMemset(c->act, 0, L * S * T * I / 2 * 8), "hipMemset");
        // phase counters and flags per launch layer: up to L * kMaxTokens with interleaved chains
        const size_t LV = L * kMaxTokens;
        c->counters = dalloc<uint32_t>((LV * kCountersPerLayer + 1) * kCounterGroupWords);
        c->error = dalloc<int32_t>(1);
        c->d_params = dalloc<DecodeParams>(1);
        check(hipMemset(c->counters, 0, (LV * kCountersPerLayer + 1) * kCounterGroupWords * 4), "hipMemset counters");
        c->flags = dalloc<uint32_t>(LV * kCountersPerLayer * kFlagCopies * kFlagStride);
        check(hipMemset(c->flags, 0, LV * kCountersPerLayer * kFlagCopies * kFlagStride * 4), "hipMemset flags");
        check(hipMemset(c->error, 0, 4), "hipMemset error");
        for (int t = 1; t <= kMaxTokens; ++t) c->grid[t] = decode_grid(c, t);
        // zero the banks so uninstalled layers are defined
        for (size_t l = 0; l < L; ++l) {
            check(hipMemsetAsync(c->router[l], 0, (E + 1) * H * 2, c->stream), "hipMemsetAsync");
        }
        check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        *out = c;
        return true;
    });
    if (!ok && c) {
        std::string keep = g_last_error;
        firewing_hip_destroy(c);
        g_last_error = keep;
    }
    return ok;
}

void firewing_hip_destroy(firewing_hip_context* c) {
    if (!c) return;
    if (c->last) (void)hipEventSynchronize(c->last);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    auto freev = [](std::vector<uint16_t*>& v) {
        for (auto* p : v)
            if (p) (void)hipFree(p);
        v.clear();
    };
    freev(c->router);
    freev(c->gate_up);
    freev(c->down);
    c->shared_up.clear();  // inside the shared_gate allocations
    freev(c->shared_gate);
    freev(c->shared_down);
    void* bufs[] = {c->d_layers, c->d_vlayers, c->d_weight_table, c->xin, c->xfinal, c->out, c->ids, c->scores,
                    c->sig, c->xw, c->logits, c->shared_act, c->act, c->counters, c->flags,
                    c->error, c->d_params};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    for (void* b : c->pf.owned)
        if (b) (void)hipFree(b);
    for (void* b : c->hc.owned)
        if (b) (void)hipFree(b);
    for (void* b : {(void*)c->lm.weight, (void*)c->lm.logits, (void*)c->lm.cand_key, (void*)c->lm.cand_pos,
                    (void*)c->lm.ids, (void*)c->lm.values})
        if (b) (void)hipFree(b);
    if (c->last) (void)hipEventDestroy(c->last);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char* firewing_hip_device_name(const firewing_hip_context* c) {
    return c ? c->device_name : "";
}

bool firewing_hip_install_layer(firewing_hip_context* c, size_t layer, const uint16_t* router,
                                const uint16_t* gate_up, const uint16_t* down,
                                const uint16_t* shared_gate, const uint16_t* shared_up,
                                const uint16_t* shared_down, const uint16_t* shared_expert_gate) {
    return guarded([&] {
        if (!c) return fail("install_layer: null context");
        if (layer >= c->shape.layers) return fail("install_layer: layer out of range");
        if (!router || !gate_up || !down || !shared_gate || !shared_up || !shared_down ||
            !shared_expert_gate)
            return fail("install_layer: null tensor");
        const size_t H = c->shape.hidden, I = c->shape.intermediate, E = c->shape.experts;
        const size_t Is = c->shape.shared_intermediate;
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        upload(c->router[layer], router, E * H * 2, s);
        upload(c->router[layer] + E * H, shared_expert_gate, H * 2, s);
        upload(c->gate_up[layer], gate_up, E * 2 * I * H * 2, s);
        upload(c->down[layer], down, E * H * I * 2, s);
        upload(c->shared_gate[layer], shared_gate, Is * H * 2, s);
        upload(c->shared_up[layer], shared_up, Is * H * 2, s);
        upload(c->shared_down[layer], shared_down, H * Is * 2, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

namespace {

// Copies byte ranges of files into device memory through pinned staging
// buffers: while one buffer's copy to HBM is in flight on the stream, the next
// is filled by parallel preads (a page-cached or NVMe file is read faster by
// several threads than by one).
class FileStreamer {
   public:
    static constexpr size_t kChunk = 32u << 20;
    static constexpr int kBuffers = 3;
    static constexpr int kReaders = 4;

    explicit FileStreamer(hipStream_t s) : s_(s) {
        for (int i = 0; i < kBuffers; ++i) {
            check(hipHostMalloc(&buf_[i], kChunk, hipHostMallocDefault), "hipHostMalloc staging");
            check(hipEventCreateWithFlags(&done_[i], hipEventDisableTiming), "hipEventCreate");
        }
    }
    ~FileStreamer() {
        (void)hipStreamSynchronize(s_);
        for (int i = 0; i < kBuffers; ++i) {
            if (done_[i]) (void)hipEventDestroy(done_[i]);
            if (buf_[i]) (void)hipHostFree(buf_[i]);
        }
        if (fd_ >= 0) ::close(fd_);
    }
    FileStreamer(const FileStreamer&) = delete;
    FileStreamer& operator=(const FileStreamer&) = delete;

    void copy(const std::string& file, uint64_t offset, uint64_t bytes, void* dst) {
        open(file);
        auto* d = static_cast<char*>(dst);
        while (bytes) {
            const size_t n = (size_t)std::min<uint64_t>(bytes, kChunk);
            const int b = next_++ % kBuffers;
            if (used_[b]) check(hipEventSynchronize(done_[b]), "hipEventSynchronize staging");
            fill(static_cast<char*>(buf_[b]), n, offset);
            check(hipMemcpyAsync(d, buf_[b], n, hipMemcpyHostToDevice, s_), "hipMemcpyAsync staging");
            check(hipEventRecord(done_[b], s_), "hipEventRecord staging");
            used_[b] = true;
            d += n;
            offset += n;
            bytes -= n;
        }
    }

   private:
    void open(const std::string& file) {
        if (file == file_) return;
        if (fd_ >= 0) ::close(fd_);
        fd_ = ::open(file.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd_ < 0) throw std::runtime_error(file + ": cannot open");
        file_ = file;
    }
    void fill(char* dst, size_t n, uint64_t offset) {
        const size_t part = (n + kReaders - 1) / kReaders;
        std::atomic<bool> short_read{false};
        auto read_part = [&](size_t lo, size_t hi) {
            while (lo < hi) {
                ssize_t got = ::pread(fd_, dst + lo, hi - lo, (off_t)(offset + lo));
                if (got <= 0) {
                    short_read = true;
                    return;
                }
                lo += (size_t)got;
            }
        };
        std::vector<std::thread> readers;
        for (size_t lo = part; lo < n; lo += part) readers.emplace_back(read_part, lo, std::min(n, lo + part));
        read_part(0, std::min(n, part));
        for (auto& t : readers) t.join();
        if (short_read) throw std::runtime_error(file_ + ": short read");
    }

    hipStream_t s_;
    void* buf_[kBuffers] = {};
    hipEvent_t done_[kBuffers] = {};
    bool used_[kBuffers] = {};
    int next_ = 0;
    int fd_ = -1;
    std::string file_;
};

}  // namespace

bool firewing_hip_safetensors_layer_plan(const firewing_hip_shape* shape, const char* path, const char* layer_prefix,
                                         firewing_hip_tensor_span* spans) {
    return guarded([&] {
        if (!shape || !path || !layer_prefix || !spans) return fail("safetensors_layer_plan: null pointer");
        fw::st::Checkpoint ckpt(path);
        auto plan = fw::st::layer_plan(ckpt, layer_prefix, shape->hidden, shape->intermediate, shape->experts,
                                       shape->shared_intermediate);
        std::vector<std::string> files;
        for (size_t i = 0; i < plan.size(); ++i) {
            auto it = std::find(files.begin(), files.end(), plan[i].file);
            if (it == files.end()) it = files.insert(files.end(), plan[i].file);
            spans[i].offset = plan[i].offset;
            spans[i].bytes = plan[i].bytes;
            spans[i].shard = (uint32_t)(it - files.begin());
        }
        return true;
    });
}

bool firewing_hip_load_layer_safetensors(firewing_hip_context* c, size_t layer, const char* path,
                                         const char* layer_prefix) {
    return guarded([&] {
        if (!c) return fail("load_layer_safetensors: null context");
        if (!path || !layer_prefix) return fail("load_layer_safetensors: null path or prefix");
        if (layer >= c->shape.layers) return fail("load_layer_safetensors: layer out of range");
        const size_t H = c->shape.hidden, E = c->shape.experts;
        // every tensor is resolved and validated before the first byte moves
        fw::st::Checkpoint ckpt(path);
        auto plan = fw::st::layer_plan(ckpt, layer_prefix, H, c->shape.intermediate, E, c->shape.shared_intermediate);
        uint16_t* dst[7] = {c->router[layer],      c->gate_up[layer],   c->down[layer],
                            c->shared_gate[layer], c->shared_up[layer], c->shared_down[layer],
                            c->router[layer] + E * H};
        Ordered ordered(c, nullptr);
        FileStreamer streamer(ordered.s);
        for (size_t i = 0; i < plan.size(); ++i) streamer.copy(plan[i].file, plan[i].offset, plan[i].bytes, dst[i]);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_generate_layers(firewing_hip_context* c, size_t first, size_t count,
                                  uint64_t seed, bool bias_feature) {
    return guarded([&] {
        if (!c) return fail("generate_layers: null context");
        if (first > c->shape.layers || count > c->shape.layers - first)
            return fail("generate_layers: layer range out of bounds");
        const size_t H = c->shape.hidden, I = c->shape.intermediate, E = c->shape.experts;
        const size_t Is = c->shape.shared_intermediate;
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        if (!c->d_weight_table) {
            std::vector<uint16_t> table(65536);
            fw_synth_normal_table(FW_SYNTH_WEIGHT_SIGMA, table.data());
            c->d_weight_table = dalloc<uint16_t>(65536);
            check(hipMemcpy(c->d_weight_table, table.data(), 65536 * 2, hipMemcpyHostToDevice),
                  "hipMemcpy table");
        }
        auto gen = [&](uint16_t* dst, size_t n, uint32_t layer, uint32_t tensor) {
            uint64_t stream = fw_synth_stream(seed, layer, tensor);
            size_t quads = (n + 3) / 4;
            const size_t chunk = (size_t)1 << 28;  // quads per launch
            for (size_t q0 = 0; q0 < quads; q0 += chunk) {
                size_t nq = std::min(chunk, quads - q0);
                size_t e0 = q0 * 4;
                size_t ne = std::min(n - e0, nq * 4);
                hipLaunchKernelGGL(k_generate, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s,
                                   dst + e0, ne, stream, (uint64_t)e0, c->d_weight_table);
                check(hipGetLastError(), "k_generate launch");
            }
        };
        std::vector<uint16_t> bias(E);
        std::vector<uint32_t> rank(E);
        DeviceBuffer dbias(E * 2);
        for (size_t l = first; l < first + count; ++l) {
            const uint32_t li = (uint32_t)l;
            gen(c->router[l], E * H, li, FW_SYNTH_ROUTER);
            gen(c->router[l] + E * H, H, li, FW_SYNTH_SHARED_EXPERT_GATE);
            gen(c->gate_up[l], E * 2 * I * H, li, FW_SYNTH_GATE_UP);
            gen(c->down[l], E * H * I, li, FW_SYNTH_DOWN);
            gen(c->shared_gate[l], Is * H, li, FW_SYNTH_SHARED_GATE);
            gen(c->shared_up[l], Is * H, li, FW_SYNTH_SHARED_UP);
            gen(c->shared_down[l], H * Is, li, FW_SYNTH_SHARED_DOWN);
            if (bias_feature) {
                fw_synth_router_bias(seed, li, (uint32_t)E, FW_SYNTH_ZIPF_BIAS_SLOPE, rank.data(),
                                     bias.data());
                check(hipMemcpyAsync(dbias.ptr, bias.data(), E * 2, hipMemcpyHostToDevice, s),
                      "hipMemcpyAsync bias");
                hipLaunchKernelGGL(k_router_bias, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, s,
                                   c->router[l], (int)E, (int)H, dbias.as<uint16_t>());
                check(hipGetLastError(), "k_router_bias launch");
                check(hipStreamSynchronize(s), "hipStreamSynchronize");
            }
        }
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_read_tensor(firewing_hip_context* c, size_t layer, int tensor, size_t first,
                              size_t count, uint16_t* out) {
    return guarded([&] {
        if (!c || !out) return fail("read_tensor: null pointer");
        if (layer >= c->shape.layers) return fail("read_tensor: layer out of range");
        const size_t H = c->shape.hidden, I = c->shape.intermediate, E = c->shape.experts;
        const size_t Is = c->shape.shared_intermediate;
        const uint16_t* base = nullptr;
        size_t n = 0;
        switch (tensor) {
            case FW_SYNTH_ROUTER: base = c->router[layer]; n = E * H; break;
            case FW_SYNTH_GATE_UP: base = c->gate_up[layer]; n = E * 2 * I * H; break;
            case FW_SYNTH_DOWN: base = c->down[layer]; n = E * H * I; break;
            case FW_SYNTH_SHARED_GATE: base = c->shared_gate[layer]; n = Is * H; break;
            case FW_SYNTH_SHARED_UP: base = c->shared_up[layer]; n = Is * H; break;
            case FW_SYNTH_SHARED_DOWN: base = c->shared_down[layer]; n = H * Is; break;
            case FW_SYNTH_SHARED_EXPERT_GATE: base = c->router[layer] + E * H; n = H; break;
            default: return fail("read_tensor: unknown tensor id");
        }
        if (first > n || count > n - first) return fail("read_tensor: range out of bounds");
        Ordered ordered(c, nullptr);
        download(out, base + first, count * 2, ordered.s);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_route(firewing_hip_context* c, size_t layer, const uint16_t* hidden,
                        size_t tokens, int order, size_t* ids, uint16_t* scores,
                        uint16_t* logits) {
    return guarded([&] {
        if (!c || !hidden || !ids || !scores) return fail("route: null pointer");
        if (layer >= c->shape.layers) return fail("route: layer out of range");
        if (tokens == 0 || tokens > 4096) return fail("route: tokens must be in [1, 4096]");
        if (order != FIREWING_HIP_LOGITS_TREE32 && order != FIREWING_HIP_LOGITS_FOLD)
            return fail("route: unknown logit order");
        const size_t H = c->shape.hidden, E = c->shape.experts, K = c->shape.top_k;
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        DeviceBuffer dx(tokens * H * 2), dl(tokens * E * 2), dids(tokens * K * 4),
            dsc(tokens * K * 2), derr(4);
        upload(dx.ptr, hidden, tokens * H * 2, s);
        check(hipMemsetAsync(derr.ptr, 0, 4, s), "hipMemsetAsync");
        for (size_t t0 = 0; t0 < tokens; t0 += 4) {
            int T = (int)std::min<size_t>(4, tokens - t0);  // H <= 2560: <= 40 KiB of LDS
            if (order == FIREWING_HIP_LOGITS_TREE32) {
                launch_linear(c->router[layer], dx.as<uint16_t>() + t0 * H, (int)E, (int)H, T,
                              dl.as<uint16_t>() + t0 * E, s);
            } else {
                hipLaunchKernelGGL(k_linear_fold, dim3((unsigned)((E + 63) / 64)), dim3(64),
                                   (size_t)T * H * 4, s, c->router[layer],
                                   dx.as<uint16_t>() + t0 * H, (int)E, (int)H, T,
                                   dl.as<uint16_t>() + t0 * E);
                check(hipGetLastError(), "k_linear_fold launch");
            }
        }
        hipLaunchKernelGGL(k_select, dim3((unsigned)tokens), dim3(64), 0, s, dl.as<uint16_t>(),
                           (int)E, (int)K, dids.as<int32_t>(), dsc.as<uint16_t>(),
                           order == FIREWING_HIP_LOGITS_TREE32 ? 1 : 0, derr.as<int32_t>());
        check(hipGetLastError(), "k_select launch");
        std::vector<int32_t> hid(tokens * K);
        int32_t err = 0;
        download(hid.data(), dids.ptr, hid.size() * 4, s);
        download(scores, dsc.ptr, tokens * K * 2, s);
        if (logits) download(logits, dl.ptr, tokens * E * 2, s);
        download(&err, derr.ptr, 4, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        if (err == 2) return fail("decoder-layer router received unsupported logits (NaN)");
        for (size_t i = 0; i < hid.size(); ++i) ids[i] = (size_t)hid[i];
        return true;
    });
}

bool firewing_hip_mixture_bf16(firewing_hip_context* c, size_t layer, const uint16_t* hidden,
                               const size_t* experts, const uint16_t* route_weights,
                               size_t count, uint16_t* mixture) {
    return guarded([&] {
        if (!c || !hidden || !experts || !route_weights || !mixture) return fail("mixture: null pointer");
        if (layer >= c->shape.layers) return fail("mixture: layer out of range");
        if (count == 0 || count > 64) return fail("mixture: count must be in [1, 64]");
        const size_t H = c->shape.hidden, I = c->shape.intermediate, E = c->shape.experts;
        for (size_t i = 0; i < count; ++i) {
            if (experts[i] >= E) return fail("mixture: expert index is out of range");
        }
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        DeviceBuffer dx(H * 2), dgo(2 * I * 2), dact(I * 2), ddo(H * 2), dw(count * H * 2), dmix(H * 2);
        upload(dx.ptr, hidden, H * 2, s);
        for (size_t i = 0; i < count; ++i) {
            const uint16_t* gu = c->gate_up[layer] + experts[i] * 2 * I * H;
            const uint16_t* dn = c->down[layer] + experts[i] * H * I;
            launch_linear(gu, dx.as<uint16_t>(), (int)(2 * I), (int)H, 1, dgo.as<uint16_t>(), s);
            hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((I + 255) / 256)), dim3(256), 0, s,
                               dgo.as<uint16_t>(), dgo.as<uint16_t>() + I, I, dact.as<uint16_t>());
            check(hipGetLastError(), "k_swiglu launch");
            launch_linear(dn, dact.as<uint16_t>(), (int)H, (int)I, 1, ddo.as<uint16_t>(), s);
            hipLaunchKernelGGL(k_scale_bf16, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, s,
                               ddo.as<uint16_t>(), route_weights[i], H, dw.as<uint16_t>() + i * H);
            check(hipGetLastError(), "k_scale_bf16 launch");
        }
        hipLaunchKernelGGL(k_mixture, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, s,
                           dw.as<uint16_t>(), (int)count, (int)H, dmix.as<uint16_t>());
        check(hipGetLastError(), "k_mixture launch");
        download(mixture, dmix.ptr, H * 2, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

// ---- many-token block (prefill) ----

static constexpr size_t kMaxPrefillTokens = 65536;

static bool prefill_args_ok(firewing_hip_context* c, size_t layer, size_t tokens, int order, std::string* why) {
    if (!c) {
        *why = "null context";
        return false;
    }
    const firewing_hip_shape& sh = c->shape;
    if (tokens == 0 || tokens > kMaxPrefillTokens) {
        *why = "tokens must be in [1, 65536]";
        return false;
    }
    if (order != FIREWING_HIP_LOGITS_TREE32) {
        *why = "the many-token block computes the in-model (TREE32) logits only";
        return false;
    }
    if (layer >= sh.layers) {
        *why = "layer out of range";
        return false;
    }
    if (sh.hidden % 256 || sh.intermediate % 128 || sh.shared_intermediate % 128) {
        *why = "the many-token block needs hidden % 256 == 0 and intermediate sizes % 128 == 0";
        return false;
    }
    return true;
}

// Scratch for `tokens` tokens (grown, never shrunk).
// Work queued before this call (on any stream) may still use the old
// buffers: the host waits for the context's last work before freeing them.
static void prefill_reserve(firewing_hip_context* c, size_t tokens, hipStream_t s) {
    auto& f = c->pf;
    if (f.tokens >= tokens) return;
    check(hipEventSynchronize(c->last), "hipEventSynchronize");
    for (void* b : f.owned)
        if (b) (void)hipFree(b);
    f.owned.clear();
    const firewing_hip_shape& sh = c->shape;
    const size_t T = tokens, H = sh.hidden, E = sh.experts, K = sh.top_k;
    const size_t Imax = std::max(sh.intermediate, sh.shared_intermediate);
    const size_t P = T * K + T, G = E + 1, tiles = P / kPfTileM + G + 1;
    auto take = [&](auto*& ptr, size_t count) {
        using T_ = std::remove_pointer_t<std::remove_reference_t<decltype(ptr)>>;
        ptr = dalloc<T_>(count);
        f.owned.push_back(ptr);
    };
    take(f.x, T * H);
    take(f.out, T * H);
    take(f.mixture, T * H);
    take(f.logits, T * E);
    take(f.gate, T);
    take(f.scores, T * K);
    take(f.ids, T * K);
    take(f.redo, (T + kPfMxTokens - 1) / kPfMxTokens * ((G + kPfMxRows - 1) / kPfMxRows));
    take(f.act, P * Imax);
    take(f.weighted, P * H);
    take(f.g.counts, G);
    take(f.g.cursor, G);
    take(f.g.offsets, G + 1);
    take(f.g.tile_group, tiles);
    take(f.g.tile_row0, tiles);
    take(f.g.tiles, 1);
    take(f.g.pair_token, P);
    take(f.g.pair_scale, P);
    take(f.g.pair_of, T * K);
    take(f.silu, 65536);
    hipLaunchKernelGGL(k_pf_silu_lut, dim3(256), dim3(256), 0, s, f.silu);
    check(hipGetLastError(), "k_pf_silu_lut launch");
    f.tokens = tokens;
}

// The many-token block on device buffers x [T][H] -> out [T][H]; the
// selection stays in c->pf (ids, scores, logits, gate logits, mixture).
// With `marks` (7 events), an event is recorded before the router and after
// each phase: router logits, selection, grouping, gate/up GEMM, down GEMM,
// combine.
static void launch_prefill(firewing_hip_context* c, size_t layer, const uint16_t* x, size_t tokens, uint16_t* out,
                           bool keep_mixture, hipStream_t s, hipEvent_t* marks = nullptr) {
    auto mark = [&](int i) {
        if (marks) check(hipEventRecord(marks[i], s), "hipEventRecord");
    };
    auto& f = c->pf;
    const firewing_hip_shape& sh = c->shape;
    const int T = (int)tokens, H = (int)sh.hidden, E = (int)sh.experts, K = (int)sh.top_k;
    const int I = (int)sh.intermediate, Is = (int)sh.shared_intermediate, Imax = std::max(I, Is);
    const int P = T * K + T, G = E + 1, max_tiles = P / kPfTileM + G + 1;
    static bool lds_attrs = false;
    if (!lds_attrs) {
        check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_router_mx),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPfMxLds),
              "hipFuncSetAttribute router");
        check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm<kPfGateUp>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPfGemmLds),
              "hipFuncSetAttribute gate/up");
        check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm<kPfDown>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPfGemmLds),
              "hipFuncSetAttribute down");
        lds_attrs = true;
    }
    // router logits on the matrix units; tiles whose inputs could meet a
    // denormal or an overflow there are recomputed on the vector units
    mark(0);
    const int row_tiles = (G + kPfMxRows - 1) / kPfMxRows;
    const int mx_tiles = (T + kPfMxTokens - 1) / kPfMxTokens * row_tiles;
    hipLaunchKernelGGL(k_pf_router_mx, dim3((mx_tiles + 7) / 8 * 8), dim3(kPfMxThreads), kPfMxLds, s, x, T, H,
                       c->router[layer], E, f.logits, f.gate, f.redo, row_tiles);
    check(hipGetLastError(), "k_pf_router_mx launch");
    hipLaunchKernelGGL(k_pf_router, dim3((T + kPfRouterTokens - 1) / kPfRouterTokens, (G + kPfRouterRows - 1) / kPfRouterRows),
                       dim3(256), 0, s, x, T, H, c->router[layer], E, f.logits, f.gate, f.redo, row_tiles);
    check(hipGetLastError(), "k_pf_router launch");
    mark(1);
    hipLaunchKernelGGL(k_select, dim3(T), dim3(64), 0, s, f.logits, E, K, f.ids, f.scores, 1, c->error);
    check(hipGetLastError(), "k_select launch");
    mark(2);
    hipLaunchKernelGGL(k_pf_zero, dim3((G + 255) / 256), dim3(256), 0, s, f.g.counts, f.g.cursor, G);
    const int chunks = (T * K + kPfChunk - 1) / kPfChunk;
    hipLaunchKernelGGL(k_pf_count, dim3(chunks), dim3(256), 0, s, f.ids, T * K, E, f.g.counts);
    hipLaunchKernelGGL(k_pf_scan, dim3(1), dim3(1024), 0, s, f.g, E, T);
    hipLaunchKernelGGL(k_pf_scatter, dim3(chunks + (T + 255) / 256), dim3(256), 0, s, f.g, f.ids, f.scores, f.gate,
                       T, K, E);
    check(hipGetLastError(), "grouping launch");
    mark(3);
    PfGemm gu{};
    gu.a = x;
    gu.lda = H;
    gu.w_routed = c->gate_up[layer];
    gu.w_shared = c->shared_gate[layer];  // shared_up follows it in the same allocation
    gu.I = I;
    gu.Is = Is;
    gu.H = H;
    gu.E = E;
    gu.out = f.act;
    gu.ldo = Imax;
    gu.n_tiles = Imax / kPfActCols;
    gu.silu = f.silu;
    // m-tiles rounded up to the XCD count (the grid's XCD-aware order)
    const int m_grid = (max_tiles + kPfXcds - 1) / kPfXcds * kPfXcds;
    hipLaunchKernelGGL(k_pf_gemm<kPfGateUp>, dim3(m_grid * gu.n_tiles), dim3(kPfGemmThreads), kPfGemmLds, s, gu, f.g);
    check(hipGetLastError(), "k_pf_gemm gate/up launch");
    mark(4);
    PfGemm dn = gu;
    dn.a = f.act;
    dn.lda = Imax;
    dn.w_routed = c->down[layer];
    dn.w_shared = c->shared_down[layer];
    dn.out = f.weighted;
    dn.ldo = H;
    dn.n_tiles = H / kPfTileN;
    hipLaunchKernelGGL(k_pf_gemm<kPfDown>, dim3(m_grid * dn.n_tiles), dim3(kPfGemmThreads), kPfGemmLds, s, dn, f.g);
    check(hipGetLastError(), "k_pf_gemm down launch");
    mark(5);
    hipLaunchKernelGGL(k_pf_combine, dim3(T), dim3(256), 0, s, f.weighted, f.g, T, K, H, E, out,
                       keep_mixture ? f.mixture : nullptr);
    check(hipGetLastError(), "k_pf_combine launch");
    mark(6);
}

bool firewing_hip_prefill_block_dev(firewing_hip_context* c, size_t layer, const uint16_t* hidden, size_t tokens,
                                    uint16_t* out, int32_t* ids, uint16_t* scores, void* stream) {
    return guarded([&] {
        std::string why;
        if (!prefill_args_ok(c, layer, tokens, FIREWING_HIP_LOGITS_TREE32, &why)) return fail("prefill_block: " + why);
        if (!hidden || !out) return fail("prefill_block: null pointer");
        if (reinterpret_cast<uintptr_t>(hidden) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
            return fail("prefill_block: hidden and out must be 16-byte aligned");
        Ordered ordered(c, stream);
        hipStream_t s = ordered.s;
        prefill_reserve(c, tokens, s);
        const size_t K = c->shape.top_k;
        launch_prefill(c, layer, hidden, tokens, out, false, s);
        if (ids) check(hipMemcpyAsync(ids, c->pf.ids, tokens * K * 4, hipMemcpyDeviceToDevice, s), "copy ids");
        if (scores) check(hipMemcpyAsync(scores, c->pf.scores, tokens * K * 2, hipMemcpyDeviceToDevice, s), "copy scores");
        return true;
    });
}

bool firewing_hip_prefill_block_profile(firewing_hip_context* c, size_t layer, const uint16_t* hidden,
                                        size_t tokens, uint16_t* out, void* stream, double* phase_us,
                                        size_t phases) {
    return guarded([&] {
        std::string why;
        if (!prefill_args_ok(c, layer, tokens, FIREWING_HIP_LOGITS_TREE32, &why)) return fail("prefill_block: " + why);
        if (!hidden || !out || !phase_us) return fail("prefill_block_profile: null pointer");
        if (phases != 6) return fail("prefill_block_profile: phases must be 6");
        if (reinterpret_cast<uintptr_t>(hidden) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
            return fail("prefill_block: hidden and out must be 16-byte aligned");
        hipEvent_t marks[7] = {};
        struct Events {
            hipEvent_t* e;
            ~Events() {
                for (int i = 0; i < 7; ++i)
                    if (e[i]) (void)hipEventDestroy(e[i]);
            }
        } owned{marks};
        for (int i = 0; i < 7; ++i) check(hipEventCreate(&marks[i]), "hipEventCreate");
        hipStream_t s;
        {
            Ordered ordered(c, stream);
            s = ordered.s;
            prefill_reserve(c, tokens, s);
            launch_prefill(c, layer, hidden, tokens, out, false, s, marks);
        }
        check(hipEventSynchronize(marks[6]), "hipEventSynchronize");
        for (int i = 0; i < 6; ++i) {
            float ms = 0.0f;
            check(hipEventElapsedTime(&ms, marks[i], marks[i + 1]), "hipEventElapsedTime");
            phase_us[i] = 1000.0 * ms;
        }
        return true;
    });
}

bool firewing_hip_prefill_block(firewing_hip_context* c, size_t layer, const uint16_t* hidden, size_t tokens,
                                uint16_t* out, firewing_hip_block_captures* cap) {
    return guarded([&] {
        std::string why;
        if (!prefill_args_ok(c, layer, tokens, FIREWING_HIP_LOGITS_TREE32, &why)) return fail("prefill_block: " + why);
        if (!hidden || !out) return fail("prefill_block: null pointer");
        if (cap && (cap->shared_gate || cap->shared_up || cap->shared_swiglu || cap->shared_down ||
                    cap->shared_gate_logit || cap->gated_shared || cap->weighted_down))
            return fail("prefill_block: the shared-expert and weighted-down captures are taken by "
                        "firewing_hip_sparse_moe_block");
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        prefill_reserve(c, tokens, s);
        const size_t H = c->shape.hidden, E = c->shape.experts, K = c->shape.top_k;
        auto& f = c->pf;
        upload(f.x, hidden, tokens * H * 2, s);
        launch_prefill(c, layer, f.x, tokens, f.out, cap && cap->routed_mixture, s);
        if (!check_device_error(c, s)) return false;
        download(out, f.out, tokens * H * 2, s);
        if (cap) {
            if (cap->router_logits) download(cap->router_logits, f.logits, tokens * E * 2, s);
            if (cap->selected_experts) {
                std::vector<int32_t> v(tokens * K);
                download(v.data(), f.ids, v.size() * 4, s);
                check(hipStreamSynchronize(s), "hipStreamSynchronize");
                for (size_t i = 0; i < v.size(); ++i) cap->selected_experts[i] = (size_t)v[i];
            }
            if (cap->selected_scores) download(cap->selected_scores, f.scores, tokens * K * 2, s);
            if (cap->routed_mixture) download(cap->routed_mixture, f.mixture, tokens * H * 2, s);
            if (cap->shared_gate_sigmoid) {
                // the shared group's pairs follow the routed ones, in token order
                int32_t off = 0;
                download(&off, f.g.offsets + E, 4, s);
                check(hipStreamSynchronize(s), "hipStreamSynchronize");
                download(cap->shared_gate_sigmoid, f.g.pair_scale + off, tokens * 2, s);
            }
        }
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

static bool step_args_ok(firewing_hip_context* c, size_t tokens, int order, std::string* why) {
    if (!c) {
        *why = "null context";
        return false;
    }
    if (tokens == 0 || tokens > (size_t)kMaxTokens) {
        *why = "tokens must be in [1, 4] (decode and MTP verify)";
        return false;
    }
    if (order != FIREWING_HIP_LOGITS_TREE32 && order != FIREWING_HIP_LOGITS_FOLD) {
        *why = "unknown logit order";
        return false;
    }
    return true;
}

bool firewing_hip_sparse_moe_block_dev(firewing_hip_context* c, size_t layer,
                                       const uint16_t* hidden, size_t tokens, int order,
                                       uint16_t* out, void* stream) {
    return guarded([&] {
        std::string why;
        if (!step_args_ok(c, tokens, order, &why)) return fail("sparse_moe_block: " + why);
        if (!hidden || !out) return fail("sparse_moe_block: null pointer");
        if (reinterpret_cast<uintptr_t>(hidden) % 4) return fail("sparse_moe_block: hidden must be 4-byte aligned");
        if (layer >= c->shape.layers) return fail("sparse_moe_block: layer out of range");
        Ordered ordered(c, stream);
        hipStream_t s = ordered.s;
        const size_t H = c->shape.hidden;
        launch_decode(c, layer, 1, (int)tokens, order, false, false, hidden, nullptr, s);
        check(hipMemcpyAsync(out, c->out, tokens * H * 2, hipMemcpyDeviceToDevice, s), "copy output");
        return true;
    });
}

namespace {

bool wants_verifier_captures(const firewing_hip_block_captures* cap) {
    return cap && (cap->routed_mixture || cap->shared_gate || cap->shared_up || cap->shared_swiglu ||
                   cap->shared_down || cap->shared_gate_logit || cap->gated_shared || cap->weighted_down);
}

// The verifier captures of a decode block (src/expert.rs:1154-1199,
// src/decoder_layer.rs:528-586): the block's intermediate vectors, recomputed
// with the standalone exact kernels on the resident weights of `layer` for the
// T inputs at x (device), the selection (ids, scores: host, rank order) and
// shared-gate sigmoids (host) the fused kernel produced. The fused kernel keeps
// none of them; the arithmetic is the same, so they are the vectors its output
// was combined from.
void take_verifier_captures(firewing_hip_context* c, size_t layer, const uint16_t* x, size_t tokens,
                            const int32_t* ids, const uint16_t* scores, const uint16_t* sig,
                            firewing_hip_block_captures* cap, hipStream_t s) {
    const size_t H = c->shape.hidden, I = c->shape.intermediate, E = c->shape.experts;
    const size_t K = c->shape.top_k, Is = c->shape.shared_intermediate;
    const int T = (int)tokens;
    const dim3 blk(256);
    auto cover = [](size_t n) { return dim3((unsigned)((n + 255) / 256)); };
    DeviceBuffer sg(tokens * Is * 2), su(tokens * Is * 2), ss(tokens * Is * 2), sd(tokens * H * 2),
        gl(tokens * 2), gs(tokens * H * 2);
    launch_linear(c->shared_gate[layer], x, (int)Is, (int)H, T, sg.as<uint16_t>(), s);
    launch_linear(c->shared_up[layer], x, (int)Is, (int)H, T, su.as<uint16_t>(), s);
    hipLaunchKernelGGL(k_swiglu, cover(tokens * Is), blk, 0, s, sg.as<uint16_t>(), su.as<uint16_t>(),
                       tokens * Is, ss.as<uint16_t>());
    check(hipGetLastError(), "k_swiglu launch");
    launch_linear(c->shared_down[layer], ss.as<uint16_t>(), (int)H, (int)Is, T, sd.as<uint16_t>(), s);
    launch_linear(c->router[layer] + E * H, x, 1, (int)H, T, gl.as<uint16_t>(), s);  // shared_expert_gate
    for (size_t t = 0; t < tokens; ++t) {
        hipLaunchKernelGGL(k_scale_bf16, cover(H), blk, 0, s, sd.as<uint16_t>() + t * H, sig[t], H,
                           gs.as<uint16_t>() + t * H);
        check(hipGetLastError(), "k_scale_bf16 launch");
    }
    // routed experts of each token in execution (ascending id) order, then the mixture
    DeviceBuffer go(2 * I * 2), act(I * 2), dn(H * 2), wd(tokens * K * H * 2), mix(tokens * H * 2);
    for (size_t t = 0; t < tokens; ++t) {
        std::vector<size_t> rank(K);
        for (size_t r = 0; r < K; ++r) rank[r] = r;
        std::sort(rank.begin(), rank.end(), [&](size_t a, size_t b) { return ids[t * K + a] < ids[t * K + b]; });
        for (size_t n = 0; n < K; ++n) {
            const size_t e = (size_t)ids[t * K + rank[n]];
            launch_linear(c->gate_up[layer] + e * 2 * I * H, x + t * H, (int)(2 * I), (int)H, 1,
                          go.as<uint16_t>(), s);
            hipLaunchKernelGGL(k_swiglu, cover(I), blk, 0, s, go.as<uint16_t>(), go.as<uint16_t>() + I, I,
                               act.as<uint16_t>());
            check(hipGetLastError(), "k_swiglu launch");
            launch_linear(c->down[layer] + e * H * I, act.as<uint16_t>(), (int)H, (int)I, 1, dn.as<uint16_t>(), s);
            hipLaunchKernelGGL(k_scale_bf16, cover(H), blk, 0, s, dn.as<uint16_t>(), scores[t * K + rank[n]], H,
                               wd.as<uint16_t>() + (t * K + n) * H);
            check(hipGetLastError(), "k_scale_bf16 launch");
        }
        hipLaunchKernelGGL(k_mixture, cover(H), blk, 0, s, wd.as<uint16_t>() + t * K * H, (int)K, (int)H,
                           mix.as<uint16_t>() + t * H);
        check(hipGetLastError(), "k_mixture launch");
    }
    if (cap->shared_gate) download(cap->shared_gate, sg.ptr, tokens * Is * 2, s);
    if (cap->shared_up) download(cap->shared_up, su.ptr, tokens * Is * 2, s);
    if (cap->shared_swiglu) download(cap->shared_swiglu, ss.ptr, tokens * Is * 2, s);
    if (cap->shared_down) download(cap->shared_down, sd.ptr, tokens * H * 2, s);
    if (cap->shared_gate_logit) download(cap->shared_gate_logit, gl.ptr, tokens * 2, s);
    if (cap->gated_shared) download(cap->gated_shared, gs.ptr, tokens * H * 2, s);
    if (cap->weighted_down) download(cap->weighted_down, wd.ptr, tokens * K * H * 2, s);
    if (cap->routed_mixture) download(cap->routed_mixture, mix.ptr, tokens * H * 2, s);
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

}  // namespace

namespace {

// The captures of the decode block that just ran on stream s for the T inputs
// at x (device): what the fused kernel keeps (logits, selection, sigmoid), then
// the verifier captures when any is asked for. Waits for s.
void collect_block_captures(firewing_hip_context* c, size_t layer, const uint16_t* x, size_t tokens,
                            firewing_hip_block_captures* cap, hipStream_t s) {
    const size_t E = c->shape.experts, K = c->shape.top_k;
    if (cap->router_logits) {
        // tagged words: two logits in the low half of each
        const size_t words = tokens * logit_stride((int)E) / 2;
        std::vector<uint64_t> lw(words);
        download(lw.data(), c->logits, words * 8, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        for (size_t t = 0; t < tokens; ++t) {
            for (size_t e = 0; e < E; ++e) {
                const uint64_t wd = lw[(t * logit_stride((int)E) + e) / 2];
                cap->router_logits[t * E + e] = (uint16_t)(wd >> (16 * (e & 1)));
            }
        }
    }
    std::vector<int32_t> ids(tokens * K);
    std::vector<uint16_t> scores(tokens * K), sig(tokens);
    download(ids.data(), c->ids, ids.size() * 4, s);
    download(scores.data(), c->scores, tokens * K * 2, s);
    download(sig.data(), c->sig, tokens * 2, s);
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (cap->selected_experts) {
        for (size_t i = 0; i < ids.size(); ++i) cap->selected_experts[i] = (size_t)ids[i];
    }
    if (cap->selected_scores) std::copy(scores.begin(), scores.end(), cap->selected_scores);
    if (cap->shared_gate_sigmoid) std::copy(sig.begin(), sig.end(), cap->shared_gate_sigmoid);
    if (wants_verifier_captures(cap))
        take_verifier_captures(c, layer, x, tokens, ids.data(), scores.data(), sig.data(), cap, s);
}

}  // namespace

bool firewing_hip_sparse_moe_block(firewing_hip_context* c, size_t layer,
                                   const uint16_t* hidden, size_t tokens, int order,
                                   uint16_t* out, firewing_hip_block_captures* cap) {
    return guarded([&] {
        std::string why;
        if (!step_args_ok(c, tokens, order, &why)) return fail("sparse_moe_block: " + why);
        if (!hidden || !out) return fail("sparse_moe_block: null pointer");
        if (layer >= c->shape.layers) return fail("sparse_moe_block: layer out of range");
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        const size_t H = c->shape.hidden;
        upload(c->xin, hidden, tokens * H * 2, s);
        launch_decode(c, layer, 1, (int)tokens, order, false, false, c->xin, nullptr, s);
        if (!check_device_error(c, s)) return false;
        download(out, c->out, tokens * H * 2, s);
        if (cap) collect_block_captures(c, layer, c->xin, tokens, cap, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_moe_step_dev(firewing_hip_context* c, const uint16_t* hidden, size_t tokens,
                               int order, bool bias_feature, uint16_t* residual,
                               uint16_t* block_out, int32_t* ids, uint16_t* scores,
                               void* stream) {
    return guarded([&] {
        std::string why;
        if (!step_args_ok(c, tokens, order, &why)) return fail("moe_step: " + why);
        if (!hidden || !residual) return fail("moe_step: null pointer");
        if (reinterpret_cast<uintptr_t>(hidden) % 4 || reinterpret_cast<uintptr_t>(residual) % 4)
            return fail("moe_step: hidden and residual must be 4-byte aligned");
        Ordered ordered(c, stream);
        hipStream_t s = ordered.s;
        const size_t L = c->shape.layers, H = c->shape.hidden, K = c->shape.top_k;
        launch_decode(c, 0, L, (int)tokens, order, true, bias_feature, hidden, residual, s);
        if (block_out)
            check(hipMemcpyAsync(block_out, c->out, L * tokens * H * 2, hipMemcpyDeviceToDevice, s),
                  "copy block outputs");
        if (ids)
            check(hipMemcpyAsync(ids, c->ids, L * tokens * K * 4, hipMemcpyDeviceToDevice, s), "copy ids");
        if (scores)
            check(hipMemcpyAsync(scores, c->scores, L * tokens * K * 2, hipMemcpyDeviceToDevice, s),
                  "copy scores");
        return true;
    });
}

bool firewing_hip_moe_step(firewing_hip_context* c, const uint16_t* hidden, size_t tokens,
                           int order, bool bias_feature, uint16_t* residual,
                           uint16_t* block_out, int32_t* ids, uint16_t* scores) {
    return guarded([&] {
        std::string why;
        if (!step_args_ok(c, tokens, order, &why)) return fail("moe_step: " + why);
        if (!hidden || !residual) return fail("moe_step: null pointer");
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        const size_t L = c->shape.layers, H = c->shape.hidden, K = c->shape.top_k;
        upload(c->xin, hidden, tokens * H * 2, s);
        launch_decode(c, 0, L, (int)tokens, order, true, bias_feature, c->xin, c->xfinal, s);
        if (!check_device_error(c, s)) return false;
        download(residual, c->xfinal, tokens * H * 2, s);
        if (block_out) download(block_out, c->out, L * tokens * H * 2, s);
        if (ids) download(ids, c->ids, L * tokens * K * 4, s);
        if (scores) download(scores, c->scores, L * tokens * K * 2, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

#ifdef FW_DECODE_TRACE
// Profiling builds only: run one step with per-task timestamps and copy them
// out ([tasks][4]: start, dependency met, end, workgroup << 8 | kind).
extern "C" bool firewing_hip_debug_traced_step(firewing_hip_context* c, const uint16_t* hidden,
                                               size_t tokens, uint64_t* out, size_t cap,
                                               size_t* tasks) {
    return guarded([&] {
        const size_t L = c->shape.layers, H = c->shape.hidden;
        const size_t E = c->shape.experts, K = c->shape.top_k, I = c->shape.intermediate;
        const size_t Is = c->shape.shared_intermediate;
        // launch layers of one-token work when the tokens run as interleaved chains
        const size_t chains = tokens >= 2 && one_token_fused(c) ? tokens : 1;
        size_t per_layer = (E + 15) / 16 + 1 + (Is + 7) / 8 + K * (tokens / chains) * (I / 8) + H / 4;
        size_t n = L * chains * per_layer;
        if (cap < n * kTraceWords) return fail("trace buffer too small");
        c->trace = dalloc<uint64_t>(n * kTraceWords);
        check(hipMemset(c->trace, 0, n * kTraceWords * 8), "hipMemset trace");
        Ordered ordered(c, nullptr);
        upload(c->xin, hidden, tokens * H * 2, ordered.s);
        launch_decode(c, 0, L, (int)tokens, 0, true, true, c->xin, nullptr, ordered.s);
        bool ok = check_device_error(c, ordered.s);
        download(out, c->trace, n * kTraceWords * 8, ordered.s);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        (void)hipFree(c->trace);
        c->trace = nullptr;
        *tasks = n;
        return ok;
    });
}
#endif

size_t firewing_hip_token_chains(const firewing_hip_context* c, size_t tokens) {
    if (!c) return 0;
    return tokens >= 2 && one_token_fused(c) ? tokens : 1;
}

bool firewing_hip_synchronize(firewing_hip_context* c) {
    return guarded([&] {
        if (!c) return fail("synchronize: null context");
        Ordered ordered(c, nullptr);  // c->stream waits for the last work on any stream
        return check_device_error(c, ordered.s);
    });
}

bool firewing_hip_set_wait_timeout(firewing_hip_context* c, double seconds) {
    return guarded([&] {
        if (!c) return fail("set_wait_timeout: null context");
        if (!(seconds > 0.0 && seconds <= 600.0)) return fail("set_wait_timeout: seconds must be in (0, 600]");
        c->timeout_seconds = seconds;
        return true;
    });
}

}  // extern "C"

// ---- hyper-connection and the in-model MoE sublayer ----

namespace {

struct HyperWeights {
    const uint16_t *norm, *down, *up, *inject;  // inject may be null (final mixer)
    int S, W, R;
};

struct HyperBuffers {
    uint16_t *normed, *mix_down, *scaled, *silu, *mix_up, *input_mix, *products, *mixed;
    uint16_t *inject, *inject_scaled, *inject_sigmoid, *weights;
};

bool hyper_shape_ok(size_t S, size_t W, size_t R, std::string* why) {
    if (S == 0 || S > 64 || W == 0 || R == 0) {
        *why = "streams must be in [1, 64], width and lowrank nonzero";
        return false;
    }
    if (S * W > 16384 || (S * W) % 2 || R > 16384 || R % 2) {
        *why = "streams * width and lowrank must be even and <= 16384";
        return false;
    }
    return true;
}

// run_hyper_connection (src/hyper_connection.rs:412-490) for T tokens at x
// ([T][S*W], device) into b, on stream s.
void queue_hyper_connection(const HyperWeights& w, const uint16_t* x, int T, const HyperBuffers& b, hipStream_t s) {
    const int SW = w.S * w.W;
    hipLaunchKernelGGL(k_hc_norm, dim3((unsigned)w.S, (unsigned)T), dim3(256), (size_t)w.W * sizeof(float), s, x,
                       w.norm, w.S, w.W, b.normed);
    check(hipGetLastError(), "k_hc_norm launch");
    for (int t = 0; t < T; ++t) {  // one token per launch: 4 * S * W bytes of LDS
        launch_linear(w.down, b.normed + (size_t)t * SW, w.R, SW, 1, b.mix_down + (size_t)t * w.R, s);
        if (w.inject) launch_linear(w.inject, b.normed + (size_t)t * SW, w.S, SW, 1, b.inject + (size_t)t * w.S, s);
    }
    hipLaunchKernelGGL(k_hc_scale_silu, dim3((unsigned)((T * w.R + 255) / 256)), dim3(256), 0, s, b.mix_down,
                       T * w.R, w.S, b.scaled, b.silu);
    check(hipGetLastError(), "k_hc_scale_silu launch");
    for (int t0 = 0; t0 < T; t0 += 4) {
        const int n = std::min(4, T - t0);
        launch_linear(w.up, b.silu + (size_t)t0 * w.R, SW, w.R, n, b.mix_up + (size_t)t0 * SW, s);
    }
    hipLaunchKernelGGL(k_hc_mix, dim3((unsigned)((w.W + 255) / 256), (unsigned)T), dim3(256), 0, s, b.mix_up,
                       b.normed, w.inject ? b.inject : nullptr, w.S, w.W, b.input_mix, b.products, b.mixed,
                       b.inject_scaled, b.inject_sigmoid, b.weights);
    check(hipGetLastError(), "k_hc_mix launch");
}

void queue_inject_residual(const uint16_t* post, const uint16_t* moe, const uint16_t* weights, int T, int S, int W,
                           uint16_t* products, uint16_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_inject_residual, dim3((unsigned)((S * W + 255) / 256), (unsigned)T), dim3(256), 0, s, post,
                       moe, weights, S, W, products, out);
    check(hipGetLastError(), "k_inject_residual launch");
}

}  // namespace

bool firewing_hip_hyper_connection_bf16(const uint16_t* input, size_t tokens, const uint16_t* hc_norm,
                                        const uint16_t* mix_down_weight, const uint16_t* mix_up_weight,
                                        const uint16_t* inject_weight, size_t streams, size_t width, size_t lowrank,
                                        firewing_hip_hyper_outputs* o) {
    return guarded([&] {
        if (!input || !hc_norm || !mix_down_weight || !mix_up_weight || !o)
            return fail("hyper_connection: null pointer");
        std::string why;
        if (!hyper_shape_ok(streams, width, lowrank, &why)) return fail("hyper_connection: " + why);
        if (tokens == 0 || tokens > 65535) return fail("hyper_connection: tokens must be in [1, 65535]");
        const size_t S = streams, W = width, R = lowrank, SW = S * W, T = tokens;
        DeviceBuffer dn(SW * 2), dd(R * SW * 2), du(SW * R * 2), di(inject_weight ? S * SW * 2 : 0), dx(T * SW * 2);
        upload(dn.ptr, hc_norm, SW * 2, nullptr);
        upload(dd.ptr, mix_down_weight, R * SW * 2, nullptr);
        upload(du.ptr, mix_up_weight, SW * R * 2, nullptr);
        if (inject_weight) upload(di.ptr, inject_weight, S * SW * 2, nullptr);
        upload(dx.ptr, input, T * SW * 2, nullptr);
        DeviceBuffer b_normed(T * SW * 2), b_md(T * R * 2), b_sc(T * R * 2), b_si(T * R * 2), b_mu(T * SW * 2),
            b_im(T * SW * 2), b_pr(T * SW * 2), b_mx(T * W * 2), b_in(T * S * 2), b_is(T * S * 2), b_ig(T * S * 2),
            b_w(T * S * 2);
        HyperBuffers b{b_normed.as<uint16_t>(), b_md.as<uint16_t>(), b_sc.as<uint16_t>(), b_si.as<uint16_t>(),
                       b_mu.as<uint16_t>(),     b_im.as<uint16_t>(), b_pr.as<uint16_t>(), b_mx.as<uint16_t>(),
                       b_in.as<uint16_t>(),     b_is.as<uint16_t>(), b_ig.as<uint16_t>(), b_w.as<uint16_t>()};
        HyperWeights w{dn.as<uint16_t>(), dd.as<uint16_t>(), du.as<uint16_t>(),
                       inject_weight ? di.as<uint16_t>() : nullptr, (int)S, (int)W, (int)R};
        queue_hyper_connection(w, dx.as<uint16_t>(), (int)T, b, nullptr);
        auto get = [&](uint16_t* dst, const uint16_t* src, size_t n) {
            if (dst) download(dst, src, n * 2, nullptr);
        };
        get(o->hyper_input_normed, b.normed, T * SW);
        get(o->mix_down, b.mix_down, T * R);
        get(o->mix_down_scaled, b.scaled, T * R);
        get(o->mix_down_silu, b.silu, T * R);
        get(o->mix_up, b.mix_up, T * SW);
        get(o->input_mix, b.input_mix, T * SW);
        get(o->products, b.products, T * SW);
        get(o->mixed, b.mixed, T * W);
        if (inject_weight) {
            get(o->inject, b.inject, T * S);
            get(o->inject_scaled, b.inject_scaled, T * S);
            get(o->inject_sigmoid, b.inject_sigmoid, T * S);
            get(o->injection_weights, b.weights, T * S);
        }
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_inject_residual_bf16(const uint16_t* post_attention, const uint16_t* moe_output,
                                       const uint16_t* injection_weights, size_t tokens, size_t streams,
                                       size_t width, uint16_t* products, uint16_t* layer_output) {
    return guarded([&] {
        if (!post_attention || !moe_output || !injection_weights || !layer_output)
            return fail("inject_residual: null pointer");
        if (streams == 0 || streams > 64 || width == 0 || streams * width > (1u << 24) || tokens == 0 ||
            tokens > 65535)
            return fail("inject_residual: invalid shape");
        const size_t T = tokens, S = streams, W = width;
        DeviceBuffer dp(T * S * W * 2), dm(T * W * 2), dw(T * S * 2), dpr(T * S * W * 2), dout(T * S * W * 2);
        upload(dp.ptr, post_attention, T * S * W * 2, nullptr);
        upload(dm.ptr, moe_output, T * W * 2, nullptr);
        upload(dw.ptr, injection_weights, T * S * 2, nullptr);
        queue_inject_residual(dp.as<uint16_t>(), dm.as<uint16_t>(), dw.as<uint16_t>(), (int)T, (int)S, (int)W,
                              dpr.as<uint16_t>(), dout.as<uint16_t>(), nullptr);
        if (products) download(products, dpr.ptr, T * S * W * 2, nullptr);
        download(layer_output, dout.ptr, T * S * W * 2, nullptr);
        check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return true;
    });
}

namespace {

// Reserve the context's hyper-connection storage: the shape on first use
// (the same for every layer), the scratch for T <= 4, and `layer`'s weights.
void hyper_reserve(firewing_hip_context* c, size_t layer, size_t streams, size_t lowrank) {
    auto& h = c->hc;
    const size_t L = c->shape.layers, H = c->shape.hidden, S = streams, R = lowrank, SW = S * H, T = kMaxTokens;
    if (h.streams == 0) {
        std::string why;
        if (!hyper_shape_ok(S, H, R, &why)) throw std::runtime_error("hyper-connection: " + why);
        h.norm.assign(L, nullptr);
        h.down.assign(L, nullptr);
        h.up.assign(L, nullptr);
        h.inject.assign(L, nullptr);
        auto take = [&](size_t n) {
            uint16_t* p = dalloc<uint16_t>(n);
            h.owned.push_back(p);
            return p;
        };
        h.normed = take(T * SW);
        h.mix_down = take(T * R);
        h.scaled = take(T * R);
        h.silu = take(T * R);
        h.mix_up = take(T * SW);
        h.input_mix = take(T * SW);
        h.products = take(T * SW);
        h.mixed = take(T * H);
        h.inject_out = take(T * S);
        h.inject_scaled = take(T * S);
        h.inject_sigmoid = take(T * S);
        h.weights = take(T * S);
        h.post = take(T * SW);
        h.layer_out = take(T * SW);
        h.inj_products = take(T * SW);
        h.streams = (int)S;
        h.lowrank = (int)R;
    } else if ((size_t)h.streams != S || (size_t)h.lowrank != R) {
        throw std::runtime_error("hyper-connection: streams and lowrank must be the same for every layer");
    }
    if (!h.norm[layer]) {
        auto take = [&](size_t n) {
            uint16_t* p = dalloc<uint16_t>(n);
            h.owned.push_back(p);
            return p;
        };
        h.norm[layer] = take(SW);
        h.down[layer] = take(R * SW);
        h.up[layer] = take(SW * R);
        h.inject[layer] = take(S * SW);
    }
}

HyperBuffers hyper_buffers(firewing_hip_context* c) {
    auto& h = c->hc;
    return HyperBuffers{h.normed, h.mix_down,  h.scaled,     h.silu,          h.mix_up,         h.input_mix,
                        h.products, h.mixed, h.inject_out, h.inject_scaled, h.inject_sigmoid, h.weights};
}

}  // namespace

bool firewing_hip_install_hyper_connection(firewing_hip_context* c, size_t layer, size_t streams, size_t lowrank,
                                           const uint16_t* hc_norm, const uint16_t* mix_down_weight,
                                           const uint16_t* mix_up_weight, const uint16_t* inject_weight) {
    return guarded([&] {
        if (!c) return fail("install_hyper_connection: null context");
        if (layer >= c->shape.layers) return fail("install_hyper_connection: layer out of range");
        if (!hc_norm || !mix_down_weight || !mix_up_weight || !inject_weight)
            return fail("install_hyper_connection: null tensor");
        Ordered ordered(c, nullptr);
        hyper_reserve(c, layer, streams, lowrank);
        const size_t SW = streams * c->shape.hidden, R = lowrank;
        auto& h = c->hc;
        upload(h.norm[layer], hc_norm, SW * 2, ordered.s);
        upload(h.down[layer], mix_down_weight, R * SW * 2, ordered.s);
        upload(h.up[layer], mix_up_weight, SW * R * 2, ordered.s);
        upload(h.inject[layer], inject_weight, streams * SW * 2, ordered.s);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_load_hyper_connection_safetensors(firewing_hip_context* c, size_t layer, size_t streams,
                                                    size_t lowrank, const char* path, const char* layer_prefix) {
    return guarded([&] {
        if (!c) return fail("load_hyper_connection_safetensors: null context");
        if (!path || !layer_prefix) return fail("load_hyper_connection_safetensors: null path or prefix");
        if (layer >= c->shape.layers) return fail("load_hyper_connection_safetensors: layer out of range");
        std::string why;
        if (!hyper_shape_ok(streams, c->shape.hidden, lowrank, &why))
            return fail("load_hyper_connection_safetensors: " + why);
        const uint64_t S = streams, SW = streams * c->shape.hidden, R = lowrank;
        fw::st::Checkpoint ckpt(path);
        const std::string pre = std::string(layer_prefix) + ".mlp_hyper_connection.";
        const std::pair<const char*, std::vector<uint64_t>> wanted[4] = {
            {"hc_norm.weight", {SW}},
            {"input_mix_weight_down.weight", {R, SW}},
            {"input_mix_weight_up.weight", {SW, R}},
            {"block_inject_weight.weight", {S, SW}},
        };
        std::vector<fw::st::Span> plan;
        for (const auto& [suffix, shape] : wanted) {
            fw::st::Span sp;
            const auto& t = ckpt.bf16(pre + suffix, shape, &sp.file);
            sp.offset = t.offset;
            sp.bytes = t.bytes;
            plan.push_back(sp);
        }
        Ordered ordered(c, nullptr);
        hyper_reserve(c, layer, streams, lowrank);
        auto& h = c->hc;
        uint16_t* dst[4] = {h.norm[layer], h.down[layer], h.up[layer], h.inject[layer]};
        FileStreamer streamer(ordered.s);
        for (size_t i = 0; i < 4; ++i) streamer.copy(plan[i].file, plan[i].offset, plan[i].bytes, dst[i]);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

namespace {

bool sublayer_args_ok(firewing_hip_context* c, size_t layer, size_t tokens, int order, std::string* why) {
    if (!step_args_ok(c, tokens, order, why)) return false;
    if (layer >= c->shape.layers) {
        *why = "layer out of range";
        return false;
    }
    if (c->hc.streams == 0 || !c->hc.norm[layer]) {
        *why = "the layer's hyper-connection is not installed";
        return false;
    }
    return true;
}

// hyper-connection -> block on its mixed input -> injection into the streams,
// all on stream s; post [T][S*H] and out [T][S*H] in device memory.
void queue_sublayer(firewing_hip_context* c, size_t layer, const uint16_t* post, int T, int order, uint16_t* out,
                    hipStream_t s) {
    auto& h = c->hc;
    const int H = (int)c->shape.hidden;
    HyperWeights w{h.norm[layer], h.down[layer], h.up[layer], h.inject[layer], h.streams, H, h.lowrank};
    queue_hyper_connection(w, post, T, hyper_buffers(c), s);
    launch_decode(c, layer, 1, T, order, false, false, h.mixed, nullptr, s);
    queue_inject_residual(post, c->out, h.weights, T, h.streams, H, h.inj_products, out, s);
}

}  // namespace

bool firewing_hip_moe_sublayer_dev(firewing_hip_context* c, size_t layer, const uint16_t* post_attention,
                                   size_t tokens, int order, uint16_t* layer_output, void* stream) {
    return guarded([&] {
        std::string why;
        if (!sublayer_args_ok(c, layer, tokens, order, &why)) return fail("moe_sublayer: " + why);
        if (!post_attention || !layer_output) return fail("moe_sublayer: null pointer");
        if (reinterpret_cast<uintptr_t>(post_attention) % 4 || reinterpret_cast<uintptr_t>(layer_output) % 4)
            return fail("moe_sublayer: post_attention and layer_output must be 4-byte aligned");
        Ordered ordered(c, stream);
        queue_sublayer(c, layer, post_attention, (int)tokens, order, layer_output, ordered.s);
        return true;
    });
}

bool firewing_hip_moe_sublayer(firewing_hip_context* c, size_t layer, const uint16_t* post_attention,
                               size_t tokens, int order, uint16_t* layer_output,
                               firewing_hip_sublayer_captures* cap) {
    return guarded([&] {
        std::string why;
        if (!sublayer_args_ok(c, layer, tokens, order, &why)) return fail("moe_sublayer: " + why);
        if (!post_attention || !layer_output) return fail("moe_sublayer: null pointer");
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        auto& h = c->hc;
        const size_t T = tokens, H = c->shape.hidden, S = h.streams, R = h.lowrank, SW = S * H;
        upload(h.post, post_attention, T * SW * 2, s);
        queue_sublayer(c, layer, h.post, (int)T, order, h.layer_out, s);
        if (!check_device_error(c, s)) return false;
        download(layer_output, h.layer_out, T * SW * 2, s);
        if (cap) {
            auto get = [&](uint16_t* dst, const uint16_t* src, size_t n) {
                if (dst) download(dst, src, n * 2, s);
            };
            firewing_hip_hyper_outputs& o = cap->hyper;
            get(o.hyper_input_normed, h.normed, T * SW);
            get(o.mix_down, h.mix_down, T * R);
            get(o.mix_down_scaled, h.scaled, T * R);
            get(o.mix_down_silu, h.silu, T * R);
            get(o.mix_up, h.mix_up, T * SW);
            get(o.input_mix, h.input_mix, T * SW);
            get(o.products, h.products, T * SW);
            get(o.mixed, h.mixed, T * H);
            get(o.inject, h.inject_out, T * S);
            get(o.inject_scaled, h.inject_scaled, T * S);
            get(o.inject_sigmoid, h.inject_sigmoid, T * S);
            get(o.injection_weights, h.weights, T * S);
            get(cap->moe_output, c->out, T * H);
            get(cap->mlp_injection_products, h.inj_products, T * SW);
            collect_block_captures(c, layer, h.mixed, T, &cap->block, s);
        }
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return true;
    });
}

// ---- LM head ----

namespace {

constexpr int kMaxLmTopK = 64;

// (Re)allocate the head for `vocab` rows; waits for the context's last work
// before freeing anything.
void lm_reserve(firewing_hip_context* c, size_t vocab) {
    auto& m = c->lm;
    if (m.vocab == vocab && m.weight) return;
    if (m.weight) check(hipEventSynchronize(c->last), "hipEventSynchronize");
    for (void* b : {(void*)m.weight, (void*)m.logits, (void*)m.cand_key, (void*)m.cand_pos, (void*)m.ids,
                    (void*)m.values})
        if (b) (void)hipFree(b);
    m = firewing_hip_context::LmHead{};
    const size_t H = c->shape.hidden, T = kMaxTokens;
    const size_t chunks = (vocab + kTopkChunk - 1) / kTopkChunk;
    m.weight = dalloc<uint16_t>(vocab * H + kLineSharePad / 2);
    m.logits = dalloc<uint16_t>(T * vocab);
    m.cand_key = dalloc<uint16_t>(T * chunks * kMaxLmTopK);
    m.cand_pos = dalloc<uint16_t>(T * chunks * kMaxLmTopK);
    m.ids = dalloc<int32_t>(T * kMaxLmTopK);
    m.values = dalloc<uint16_t>(T * kMaxLmTopK);
    m.vocab = vocab;
}

bool lm_args_ok(firewing_hip_context* c, size_t vocab, std::string* why) {
    if (!c) {
        *why = "null context";
        return false;
    }
    if (vocab == 0 || vocab > (size_t)INT32_MAX / 8 || vocab * c->shape.hidden * 2 > ((size_t)1 << 33)) {
        *why = "vocab must be in [1, 2^28) with the head below 8 GiB";
        return false;
    }
    return true;
}

template <int NT>
const void* lm_kernel(bool wide) {
    return wide ? reinterpret_cast<const void*>(&k_lm_head<NT, 80>) : reinterpret_cast<const void*>(&k_lm_head<NT, 64>);
}

const void* lm_kernel_for(int T, bool wide) {
    switch (T) {
        case 1: return lm_kernel<1>(wide);
        case 2: return lm_kernel<2>(wide);
        case 3: return lm_kernel<3>(wide);
        default: return lm_kernel<4>(wide);
    }
}

// logits [T][V] (scratch when null), then the top-k ids and values, on stream s.
void queue_lm_head(firewing_hip_context* c, const uint16_t* x, int T, int k, uint16_t* logits, int32_t* ids,
                   uint16_t* values, hipStream_t s) {
    auto& m = c->lm;
    const int V = (int)m.vocab, H = (int)c->shape.hidden;
    const bool wide = H > 2048;
    const void* fn = lm_kernel_for(T, wide);
    if (m.grid == 0) {
        int per_cu = 0;
        check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, (size_t)kMaxTokens * H * 4),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
        m.grid = std::max(1, per_cu) * c->cu_count;
    }
    uint16_t* out = logits ? logits : m.logits;
    const uint16_t* w = m.weight;
    void* args[] = {&w, &x, (void*)&V, (void*)&H, &out};
    check(hipLaunchKernel(fn, dim3((unsigned)m.grid), dim3(256), args, (size_t)T * H * 4, s), "k_lm_head launch");
    const int chunks = (V + kTopkChunk - 1) / kTopkChunk;
    hipLaunchKernelGGL(k_lm_topk_chunks, dim3((unsigned)chunks, (unsigned)T), dim3(256), 0, s, out, V, k, m.cand_key,
                       m.cand_pos);
    check(hipGetLastError(), "k_lm_topk_chunks launch");
    // the merge's candidates a lane: the fewest that hold chunks * k
    const int n = chunks * k;
    if (n <= 256 * 8)
        hipLaunchKernelGGL(k_lm_topk_merge<8>, dim3((unsigned)T), dim3(256), 0, s, m.cand_key, m.cand_pos, n, k, ids,
                           values);
    else if (n <= 256 * 16)
        hipLaunchKernelGGL(k_lm_topk_merge<16>, dim3((unsigned)T), dim3(256), 0, s, m.cand_key, m.cand_pos, n, k, ids,
                           values);
    else
        hipLaunchKernelGGL(k_lm_topk_merge<32>, dim3((unsigned)T), dim3(256), 0, s, m.cand_key, m.cand_pos, n, k, ids,
                           values);
    check(hipGetLastError(), "k_lm_topk_merge launch");
}

}  // namespace

bool firewing_hip_install_lm_head(firewing_hip_context* c, const uint16_t* weight, size_t vocab) {
    return guarded([&] {
        std::string why;
        if (!lm_args_ok(c, vocab, &why)) return fail("install_lm_head: " + why);
        if (!weight) return fail("install_lm_head: null weight");
        lm_reserve(c, vocab);
        Ordered ordered(c, nullptr);
        upload(c->lm.weight, weight, vocab * c->shape.hidden * 2, ordered.s);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_generate_lm_head(firewing_hip_context* c, size_t vocab, uint64_t seed) {
    return guarded([&] {
        std::string why;
        if (!lm_args_ok(c, vocab, &why)) return fail("generate_lm_head: " + why);
        lm_reserve(c, vocab);
        Ordered ordered(c, nullptr);
        if (!c->d_weight_table) {
            std::vector<uint16_t> table(65536);
            fw_synth_normal_table(FW_SYNTH_WEIGHT_SIGMA, table.data());
            c->d_weight_table = dalloc<uint16_t>(65536);
            check(hipMemcpy(c->d_weight_table, table.data(), 65536 * 2, hipMemcpyHostToDevice), "hipMemcpy table");
        }
        const size_t n = vocab * c->shape.hidden;
        const uint64_t stream = fw_synth_stream(seed, 0, FW_SYNTH_LM_HEAD);
        const size_t quads = (n + 3) / 4;
        hipLaunchKernelGGL(k_generate, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, ordered.s, c->lm.weight, n,
                           stream, (uint64_t)0, (const uint16_t*)c->d_weight_table);
        check(hipGetLastError(), "k_generate launch");
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_load_lm_head_safetensors(firewing_hip_context* c, const char* path, const char* tensor,
                                           size_t vocab) {
    return guarded([&] {
        std::string why;
        if (!lm_args_ok(c, vocab, &why)) return fail("load_lm_head_safetensors: " + why);
        if (!path || !tensor) return fail("load_lm_head_safetensors: null path or tensor name");
        fw::st::Checkpoint ckpt(path);
        fw::st::Span sp;
        const auto& t = ckpt.bf16(tensor, {(uint64_t)vocab, (uint64_t)c->shape.hidden}, &sp.file);
        lm_reserve(c, vocab);
        Ordered ordered(c, nullptr);
        FileStreamer streamer(ordered.s);
        streamer.copy(sp.file, t.offset, t.bytes, c->lm.weight);
        check(hipStreamSynchronize(ordered.s), "hipStreamSynchronize");
        return true;
    });
}

bool firewing_hip_lm_head_dev(firewing_hip_context* c, const uint16_t* hidden, size_t tokens, size_t k,
                              uint16_t* logits, int32_t* ids, uint16_t* values, void* stream) {
    return guarded([&] {
        if (!c) return fail("lm_head: null context");
        if (!c->lm.weight) return fail("lm_head: no LM head installed");
        if (tokens == 0 || tokens > (size_t)kMaxTokens) return fail("lm_head: tokens must be in [1, 4]");
        if (k == 0 || k > (size_t)kMaxLmTopK || k > c->lm.vocab) return fail("lm_head: k must be in [1, min(64, vocab)]");
        if ((c->lm.vocab + kTopkChunk - 1) / kTopkChunk * k > 8192)
            return fail("lm_head: ceil(vocab / 4096) * k must be <= 8192");
        if (!hidden || !ids || !values) return fail("lm_head: null pointer");
        Ordered ordered(c, stream);
        queue_lm_head(c, hidden, (int)tokens, (int)k, logits, ids, values, ordered.s);
        return true;
    });
}

bool firewing_hip_lm_head(firewing_hip_context* c, const uint16_t* hidden, size_t tokens, size_t k,
                          uint16_t* logits, size_t* ids, uint16_t* values) {
    return guarded([&] {
        if (!c) return fail("lm_head: null context");
        if (!c->lm.weight) return fail("lm_head: no LM head installed");
        if (tokens == 0 || tokens > (size_t)kMaxTokens) return fail("lm_head: tokens must be in [1, 4]");
        if (k == 0 || k > (size_t)kMaxLmTopK || k > c->lm.vocab) return fail("lm_head: k must be in [1, min(64, vocab)]");
        if ((c->lm.vocab + kTopkChunk - 1) / kTopkChunk * k > 8192)
            return fail("lm_head: ceil(vocab / 4096) * k must be <= 8192");
        if (!hidden || !ids || !values) return fail("lm_head: null pointer");
        Ordered ordered(c, nullptr);
        hipStream_t s = ordered.s;
        const size_t H = c->shape.hidden, V = c->lm.vocab;
        upload(c->xin, hidden, tokens * H * 2, s);
        queue_lm_head(c, c->xin, (int)tokens, (int)k, nullptr, c->lm.ids, c->lm.values, s);
        if (logits) download(logits, c->lm.logits, tokens * V * 2, s);
        std::vector<int32_t> hid(tokens * k);
        download(hid.data(), c->lm.ids, tokens * k * 4, s);
        download(values, c->lm.values, tokens * k * 2, s);
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        for (size_t i = 0; i < hid.size(); ++i) ids[i] = (size_t)hid[i];
        return true;
    });
}

// ---- compressed expert container: GPU zstd decoding ----

struct firewing_hip_zstd_decoder {
    fw::zs::Decoder dec;
    firewing_hip_zstd_decoder(int device, size_t frames, size_t content) : dec(device, frames, content) {}
};

namespace {

const char* zstd_status_name(uint32_t s) {
    static const char* names[] = {"ok",
                                  "not a zstd frame",
                                  "unsupported or malformed frame header",
                                  "truncated frame",
                                  "malformed block",
                                  "too many blocks",
                                  "malformed literals section",
                                  "malformed Huffman table or stream",
                                  "malformed FSE table",
                                  "malformed sequences",
                                  "offset beyond the decoded bytes",
                                  "decoded size differs from the expected size",
                                  "scratch exceeded",
                                  "bytes after the frame"};
    return s < sizeof(names) / sizeof(names[0]) ? names[s] : "unknown failure";
}

// the first failed frame of a finished call, as an error; true if none failed
bool zstd_report(fw::zs::Decoder& d, uint32_t* status, size_t n) {
    std::vector<uint32_t> st, blk;
    d.statuses(&st, &blk);
    if (status) std::copy(st.begin(), st.begin() + std::min(n, st.size()), status);
    for (size_t i = 0; i < st.size(); ++i)
        if (st[i] != 0)
            return fail("zstd frame " + std::to_string(i) + ": " + zstd_status_name(st[i]) + " (block " +
                        std::to_string(blk[i]) + ")");
    return true;
}

bool zstd_jobs(const uint8_t* src, size_t src_bytes, const firewing_hip_zstd_frame* frames, size_t n,
               bool unshuffle, std::vector<fw::zs::FrameJob>* jobs) {
    jobs->resize(n);
    for (size_t i = 0; i < n; ++i) {
        const auto& f = frames[i];
        if (f.src_offset > src_bytes || f.src_bytes > src_bytes - f.src_offset)
            return fail("zstd_decode: frame " + std::to_string(i) + " lies outside the source buffer");
        (*jobs)[i] = fw::zs::FrameJob{src + f.src_offset, f.src_bytes, f.content_bytes,
                                      static_cast<uint8_t*>(f.dst), static_cast<uint8_t*>(f.dst_tail),
                                      f.split, unshuffle};
    }
    return true;
}

}  // namespace

firewing_hip_zstd_decoder* firewing_hip_zstd_create(int device, size_t max_frames, size_t max_content_bytes) {
    firewing_hip_zstd_decoder* d = nullptr;
    guarded([&] {
        d = new firewing_hip_zstd_decoder(device, max_frames, max_content_bytes);
        return true;
    });
    return d;
}

void firewing_hip_zstd_destroy(firewing_hip_zstd_decoder* d) { delete d; }

bool firewing_hip_zstd_decode_dev(firewing_hip_zstd_decoder* d, const uint8_t* src, size_t src_bytes,
                                  const firewing_hip_zstd_frame* frames, size_t n, bool bf16_unshuffle,
                                  void* stream) {
    return guarded([&] {
        if (!d) return fail("zstd_decode: null decoder");
        if (n && (!src || !frames)) return fail("zstd_decode: null pointer");
        std::vector<fw::zs::FrameJob> jobs;
        if (!zstd_jobs(src, src_bytes, frames, n, bf16_unshuffle, &jobs)) return false;
        std::string why;
        if (!d->dec.queue(jobs, static_cast<hipStream_t>(stream), &why)) return fail(why);
        return true;
    });
}

bool firewing_hip_zstd_decode(firewing_hip_zstd_decoder* d, const uint8_t* src, size_t src_bytes,
                              const firewing_hip_zstd_frame* frames, size_t n, bool bf16_unshuffle,
                              uint32_t* status) {
    return guarded([&] {
        if (!d) return fail("zstd_decode: null decoder");
        if (n && (!src || !frames)) return fail("zstd_decode: null pointer");
        check(hipSetDevice(d->dec.device()), "hipSetDevice");
        uint8_t* pin = d->dec.pinned(std::max<size_t>(src_bytes, 1));
        uint8_t* dev = d->dec.device_source(std::max<size_t>(src_bytes, 1));
        std::vector<fw::zs::FrameJob> jobs;
        if (!zstd_jobs(dev, src_bytes, frames, n, bf16_unshuffle, &jobs)) return false;
        check(hipEventSynchronize(d->dec.last()), "hipEventSynchronize");  // the staging is free
        std::memcpy(pin, src, src_bytes);
        hipStream_t s = nullptr;
        check(hipMemcpyAsync(dev, pin, src_bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
        std::string why;
        if (!d->dec.queue(jobs, s, &why)) return fail(why);
        return zstd_report(d->dec, status, n);
    });
}

bool firewing_hip_zstd_status(firewing_hip_zstd_decoder* d, uint32_t* status, size_t n) {
    return guarded([&] {
        if (!d) return fail("zstd_status: null decoder");
        return zstd_report(d->dec, status, n);
    });
}

bool firewing_hip_install_experts_zstd(firewing_hip_context* c, firewing_hip_zstd_decoder* d, size_t layer,
                                       const uint32_t* experts, size_t n, const uint8_t* src, size_t src_bytes,
                                       const uint64_t* offsets, const uint64_t* sizes) {
    return guarded([&] {
        if (!c || !d) return fail("install_experts_zstd: null context or decoder");
        if (layer >= c->shape.layers) return fail("install_experts_zstd: layer out of range");
        if (n && (!experts || !src || !offsets || !sizes)) return fail("install_experts_zstd: null pointer");
        const size_t H = c->shape.hidden, I = c->shape.intermediate, E = c->shape.experts;
        const uint64_t content = 6ull * I * H;
        if (content > d->dec.max_content()) return fail("install_experts_zstd: the decoder's max_content is below 6*I*H");
        std::vector<firewing_hip_zstd_frame> frames(n);
        for (size_t i = 0; i < n; ++i) {
            if (experts[i] >= E) return fail("install_experts_zstd: expert id out of range");
            for (size_t j = 0; j < i; ++j)
                if (experts[j] == experts[i]) return fail("install_experts_zstd: repeated expert id");
            frames[i] = firewing_hip_zstd_frame{offsets[i], sizes[i], content,
                                                c->gate_up[layer] + (size_t)experts[i] * 2 * I * H,
                                                c->down[layer] + (size_t)experts[i] * H * I, 4ull * I * H};
        }
        check(hipSetDevice(d->dec.device()), "hipSetDevice");
        if (d->dec.device() != c->device) return fail("install_experts_zstd: decoder and context on different GPUs");
        uint8_t* pin = d->dec.pinned(std::max<size_t>(src_bytes, 1));
        uint8_t* dev = d->dec.device_source(std::max<size_t>(src_bytes, 1));
        std::vector<fw::zs::FrameJob> jobs;
        if (!zstd_jobs(dev, src_bytes, frames.data(), n, true, &jobs)) return false;
        check(hipEventSynchronize(d->dec.last()), "hipEventSynchronize");
        std::memcpy(pin, src, src_bytes);
        {
            Ordered ordered(c, nullptr);
            check(hipMemcpyAsync(dev, pin, src_bytes, hipMemcpyHostToDevice, ordered.s), "hipMemcpyAsync");
            std::string why;
            if (!d->dec.queue(jobs, ordered.s, &why)) return fail(why);
        }
        return zstd_report(d->dec, nullptr, n);
    });
}
