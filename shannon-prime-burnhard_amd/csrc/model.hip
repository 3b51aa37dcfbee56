// model.hip — GPU residency of a GGUF file's weights (include/spq4k_gguf.h).
//
// spq4k_model_load plans which tensors go to the GPU the way
// LlamaWeights::load_backend_offload_ does (desktop/engine/src/
// llama_weights.cpp:483-720: layers [0, n_gpu_layers) or all of them, the
// expert-bank split at experts_on_cpu), restricted to the types the library
// runs (Q4_K, Q5_K, Q6_K, Q8_0), makes one device allocation for all of them
// (ggml_backend_alloc_ctx_tensors) and copies the bytes from the file mapping
// with two pinned staging buffers: the host fills one (several threads
// copying from the mapping) while the DMA engine drains the other
// (ggml_backend_tensor_set per tensor in the reference). Each resident tensor
// is an spq4k_weights view of the allocation.
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

#include <algorithm>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "spq4k.h"
#include "spq4k_gguf.h"

// the failure message shared with the file reader (spq4k_gguf_strerror)
namespace spq4k_gguf_detail {
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
}

namespace {

#define model_fail spq4k_gguf_detail::fail

bool runs_type(int t) {
    return t == SPQ4K_TYPE_Q4_K || t == SPQ4K_TYPE_Q5_K || t == SPQ4K_TYPE_Q6_K || t == SPQ4K_TYPE_Q8_0;
}

// layer index of a "blk.N." name, -1 for tensors outside layers
int layer_of(const char* name) {
    int L = -1, n = 0;
    if (sscanf(name, "blk.%d.%n", &L, &n) == 1 && n > 0 && L >= 0) return L;
    return -1;
}

// "blk.N.ffn_{gate,up,down}_exps.weight" (llama_weights.cpp:579-586)
bool is_exps(const char* name) {
    int L = -1, n = 0;
    for (const char* f : {"blk.%d.ffn_gate_exps.weight%n", "blk.%d.ffn_up_exps.weight%n", "blk.%d.ffn_down_exps.weight%n"}) {
        n = 0;
        if (sscanf(name, f, &L, &n) == 1 && n > 0 && name[n] == '\0') return true;
    }
    return false;
}

struct Plan {
    std::string name;
    int type;
    int64_t M, K, E;
    int base;              // first expert on the GPU
    const uint8_t* src;    // in the mapping
    size_t bytes;
    size_t off;            // in the device allocation
};

// copy n bytes with up to `threads` threads (the mapping's pages fault in
// from the page cache or the disk; several threads keep the DMA fed)
void par_copy(void* dst, const void* src, size_t n, int threads) {
    if (threads <= 1 || n < ((size_t)1 << 20)) {
        memcpy(dst, src, n);
        return;
    }
    std::vector<std::thread> th;
    const size_t part = (n / threads + 4095) & ~(size_t)4095;
    for (int i = 0; i < threads; ++i) {
        const size_t a = (size_t)i * part;
        if (a >= n) break;
        const size_t b = std::min(n, a + part);
        th.emplace_back([=] { memcpy(static_cast<uint8_t*>(dst) + a, static_cast<const uint8_t*>(src) + a, b - a); });
    }
    for (auto& t : th) t.join();
}

}  // namespace

struct spq4k_model {
    int device = 0;
    uint8_t* arena = nullptr;
    size_t bytes = 0;
    std::vector<std::string> names;
    std::vector<spq4k_weights*> weights;
    std::vector<int> bases;
    std::unordered_map<std::string, size_t> index;
};

extern "C" {

void spq4k_model_free(spq4k_model* m) {
    if (!m) return;
    for (spq4k_weights* w : m->weights) spq4k_weights_free(w);
    if (m->arena) {
        (void)hipSetDevice(m->device);
        (void)hipFree(m->arena);
    }
    delete m;
}

int spq4k_model_load(spq4k_ctx* ctx, const spq4k_gguf* g, int n_gpu_layers, int experts_on_cpu, spq4k_model** out) {
    if (!out) return model_fail(-EINVAL, "model: null out");
    *out = nullptr;
    if (!ctx || !g) return model_fail(-EINVAL, "model: null context or file");
    const int device = spq4k_get_device(ctx);
    if (device < 0) return model_fail(-EINVAL, "model: bad context");
    hipStream_t stream = (hipStream_t)spq4k_get_stream(ctx);
    const int64_t nt = spq4k_gguf_n_tensors(g);
    int n_layer = 0;
    for (int64_t i = 0; i < nt; ++i) n_layer = std::max(n_layer, layer_of(spq4k_gguf_tensor_name(g, i)) + 1);
    const bool full = n_gpu_layers < 0 || n_gpu_layers >= n_layer;

    std::vector<Plan> plan;
    size_t total = 0;
    for (int64_t i = 0; i < nt; ++i) {
        const char* name = spq4k_gguf_tensor_name(g, i);
        const int type = spq4k_gguf_tensor_type(g, i);
        int64_t ne[4];
        const int nd = spq4k_gguf_tensor_shape(g, i, ne);
        if (!runs_type(type) || nd < 2 || ne[3] != 1 || ne[0] <= 0 || ne[1] <= 0 || ne[2] <= 0) continue;
        const int L = layer_of(name);
        if (!full && !(L >= 0 && L < n_gpu_layers)) continue;
        Plan p;
        p.name = name;
        p.type = type;
        p.K = ne[0];
        p.M = ne[1];
        p.E = ne[2];
        p.base = 0;
        p.src = static_cast<const uint8_t*>(spq4k_gguf_tensor_data(g, i));
        p.bytes = spq4k_gguf_tensor_nbytes(g, i);
        if (experts_on_cpu > 0 && is_exps(name)) {
            const int64_t pivot = std::min<int64_t>(experts_on_cpu, p.E - 1);
            if (pivot > 0 && pivot < p.E && p.bytes % (size_t)p.E == 0) {
                const size_t stride = p.bytes / (size_t)p.E;
                p.base = (int)pivot;
                p.src += (size_t)pivot * stride;
                p.bytes = (size_t)(p.E - pivot) * stride;
                p.E -= pivot;
            }
        }
        p.off = total;
        total += (p.bytes + 255) & ~(size_t)255;
        plan.push_back(std::move(p));
    }

    spq4k_model* m = new (std::nothrow) spq4k_model();
    if (!m) return model_fail(-ENOMEM, "model: out of memory");
    m->device = device;
    m->bytes = total;
    if (hipSetDevice(device) != hipSuccess) {
        delete m;
        return model_fail(-EIO, "model: hipSetDevice(%d) failed", device);
    }
    if (total > 0 && hipMalloc(&m->arena, total) != hipSuccess) {
        m->arena = nullptr;
        spq4k_model_free(m);
        return model_fail(-ENOMEM, "model: device allocation of %zu bytes failed", total);
    }

    // staging: NBUF pinned buffers of STAGE MiB (SPQ4K_UPLOAD_BUFFERS,
    // SPQ4K_UPLOAD_STAGE_MB), each filled by THREADS threads
    // (SPQ4K_UPLOAD_THREADS) while the DMA engine drains the others
    constexpr int MAXBUF = 8;
    size_t stage_mb = 16;
    int nbuf = 3;
    if (const char* f = getenv("SPQ4K_UPLOAD_STAGE_MB")) {
        const long v = atol(f);
        if (v >= 1 && v <= 1024) stage_mb = (size_t)v;
    }
    if (const char* f = getenv("SPQ4K_UPLOAD_BUFFERS")) {
        const int v = atoi(f);
        if (v >= 2 && v <= MAXBUF) nbuf = v;
    }
    const size_t stage = std::min<size_t>(stage_mb << 20, std::max<size_t>(total, 4096));
    void* pin[MAXBUF] = {};
    hipEvent_t ev[MAXBUF] = {};
    bool used[MAXBUF] = {};
    int rc = 0;
    auto cleanup = [&]() {
        for (int k = 0; k < nbuf; ++k) {
            if (ev[k]) (void)hipEventDestroy(ev[k]);
            if (pin[k]) (void)hipHostFree(pin[k]);
        }
    };
    if (total > 0) {
        for (int k = 0; k < nbuf && rc == 0; ++k) {
            if (hipHostMalloc(&pin[k], stage, hipHostMallocDefault) != hipSuccess) {
                pin[k] = nullptr;
                rc = model_fail(-ENOMEM, "model: pinned staging of %zu bytes failed", stage);
            } else if (hipEventCreateWithFlags(&ev[k], hipEventDisableTiming) != hipSuccess) {
                ev[k] = nullptr;
                rc = model_fail(-EIO, "model: hipEventCreate failed");
            }
        }
        const unsigned hw = std::thread::hardware_concurrency();
        int threads = (int)std::max(1u, std::min(4u, hw ? hw : 1u));
        if (const char* f = getenv("SPQ4K_UPLOAD_THREADS")) {
            const int v = atoi(f);
            if (v >= 1 && v <= 64) threads = v;
        }
        int k = 0;
        for (size_t pi = 0; pi < plan.size() && rc == 0; ++pi) {
            const Plan& p = plan[pi];
            (void)madvise((void*)((uintptr_t)p.src & ~(uintptr_t)4095),
                          p.bytes + ((uintptr_t)p.src & 4095), MADV_WILLNEED);
            for (size_t o = 0; o < p.bytes && rc == 0; o += stage) {
                const size_t n = std::min(stage, p.bytes - o);
                if (used[k] && hipEventSynchronize(ev[k]) != hipSuccess) {
                    rc = model_fail(-EIO, "model: staging wait failed");
                    break;
                }
                par_copy(pin[k], p.src + o, n, threads);
                if (hipMemcpyAsync(m->arena + p.off + o, pin[k], n, hipMemcpyHostToDevice, stream) != hipSuccess ||
                    hipEventRecord(ev[k], stream) != hipSuccess) {
                    rc = model_fail(-EIO, "model: upload of '%s' failed", p.name.c_str());
                    break;
                }
                used[k] = true;
                k = (k + 1) % nbuf;
            }
        }
        if (hipStreamSynchronize(stream) != hipSuccess && rc == 0) rc = model_fail(-EIO, "model: upload failed");
    }
    cleanup();
    for (size_t pi = 0; pi < plan.size() && rc == 0; ++pi) {
        const Plan& p = plan[pi];
        spq4k_weights* w = nullptr;
        const int wr = spq4k_weights_wrap_type(ctx, p.type, m->arena + p.off, p.M, p.K, p.E, &w);
        if (wr) {
            rc = model_fail(wr, "model: tensor '%s': %s", p.name.c_str(), spq4k_last_error(ctx));
            break;
        }
        m->index.emplace(p.name, m->weights.size());
        m->names.push_back(p.name);
        m->weights.push_back(w);
        m->bases.push_back(p.base);
    }
    if (rc) {
        spq4k_model_free(m);
        return rc;
    }
    *out = m;
    return 0;
}

spq4k_weights* spq4k_model_weights(const spq4k_model* m, const char* name) {
    if (!m || !name) return nullptr;
    auto it = m->index.find(name);
    return it == m->index.end() ? nullptr : m->weights[it->second];
}

int spq4k_model_expert_base(const spq4k_model* m, const char* name) {
    if (!m || !name) return -1;
    auto it = m->index.find(name);
    return it == m->index.end() ? -1 : m->bases[it->second];
}

int64_t spq4k_model_n_tensors(const spq4k_model* m) { return m ? (int64_t)m->names.size() : -1; }

const char* spq4k_model_tensor_name(const spq4k_model* m, int64_t i) {
    return m && i >= 0 && (size_t)i < m->names.size() ? m->names[(size_t)i].c_str() : nullptr;
}

size_t spq4k_model_nbytes(const spq4k_model* m) { return m ? m->bytes : 0; }

}  // extern "C"
