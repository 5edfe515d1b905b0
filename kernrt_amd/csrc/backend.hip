// Host side of the KernRT HIP backend: the C ABI declared in
// include/kernrt_hip.h, over one in-order HIP stream per context.
//
// Mirrors the reference `Backend` trait (src/backends/mod.rs:264-404): the
// context owns activation buffers, weights and the KV cache; ops are enqueued
// and `kr_read` is the only barrier. Host slices (positions, slots, windows)
// are staged through pinned memory with a stream-ordered copy before the call
// returns, so callers may reuse them at once (the Metal backend could defer
// those reads to commit time; a HIP stream runs eagerly).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/kernrt_hip.h"
#include "internal.hpp"
#include "kernels.hpp"
#include "numerics.hpp"

using kr::DevMatrix;

namespace {

struct DevBuf {
    float* p = nullptr;
    size_t len = 0;
    bool live = false;
};

struct Mat {
    DevMatrix m{};
    // x86 logits over a Q8_0x4 classifier (quant.rs:223-236): -1 unknown,
    // 0 the re-quantization identity holds, 1 `requant` holds the copy.
    int requant_state = -1;
    DevMatrix requant{};
    // A Q8_0 matrix's chain-major copy for the chain-split prefill GEMM
    // (launch_gemm_q8_cs), made on its first use; the matrix never changes
    // after it is made, so the copy stays valid until the matrix is freed.
    DevMatrix cm{};
};

// A host slice staged into device memory through a pinned double buffer.
struct IdxStage {
    uint32_t* dev = nullptr;
    size_t cap = 0;
    std::vector<uint32_t> last;
    uint32_t* pinned[2] = {nullptr, nullptr};
    size_t pinned_cap = 0;
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool recorded[2] = {false, false};
    int cur = 0;
};

struct RopeTable {
    float2* dev = nullptr;
    size_t n_pos = 0;
};

// The activation workspace of kr_matmul_noalloc: a fixed device array, so
// that entry point never allocates. Each device holds its own copy from the
// first kr_open on it until the process ends. Host code must not pass
// `scratch` itself to a kernel (in host code the name is a stand-in, not a
// device address): kr_open looks up each device's address once, with that
// device current, and every use goes through that pointer.
constexpr size_t kNoAllocMaxElems = (size_t)4 << 20;  // rows * in_dim per call
constexpr size_t kScratchQuants = kNoAllocMaxElems;                        // int8 [rows][K]
constexpr size_t kScratchScales = kNoAllocMaxElems / 32 * sizeof(float);   // f32 [rows][K/32]
constexpr size_t kScratchBits = kNoAllocMaxElems / 32 * sizeof(uint16_t);  // f16 bits [rows][K/32]
constexpr size_t kScratchBytes = kScratchQuants + kScratchScales + kScratchBits;
static_assert(kScratchQuants % 256 == 0 && kScratchScales % 256 == 0, "sections stay 256-byte aligned");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_dev[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// The device address of `scratch` on `device` (current), looked up once.
hipError_t scratch_address(int device, uint8_t** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if (!g_scratch_dev[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_dev[device] = (uint8_t*)p;
    }
    *out = g_scratch_dev[device];
    return hipSuccess;
}

}  // namespace

struct kr_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint8_t* scratch = nullptr;  // this device's `scratch` array (kr_matmul_noalloc)
    std::string err;
    std::string devname;
    const char* storage = "f32";
    std::vector<DevBuf> bufs;
    std::vector<Mat*> mats;
    kr_mat embedding = KR_NO_MAT, classifier = KR_NO_MAT;
    std::vector<std::array<kr_mat, 9>> proj;
    bool prepared = false;
    size_t n_layers = 0, kv_dim = 0, seq_len = 0;
    float* kc = nullptr;
    float* vc = nullptr;
    // quantized-activation workspace
    int8_t* wq = nullptr;
    float* ws = nullptr;
    uint16_t* wh = nullptr;
    size_t cap_q = 0, cap_s = 0;
    // a second one: SiLU(gate) * up quantized by the gate/up GEMM while that
    // GEMM still reads the first
    int8_t* wq2 = nullptr;
    float* ws2 = nullptr;
    uint16_t* wh2 = nullptr;
    size_t cap_q2 = 0, cap_s2 = 0;
    float* tmp = nullptr;
    size_t cap_tmp = 0;
    IdxStage st_pos, st_slots, st_win, st_tok;
    std::map<std::pair<uint32_t, size_t>, RopeTable> rope;
    uint32_t* tokens = nullptr;
    static constexpr size_t kTokens = 1 << 16;
    unsigned int* counter = nullptr;
    // bumped whenever a buffer that captured kernels may reference moves
    // (workspace, staging, rope tables): cached HIP graphs are then stale
    uint64_t epoch = 0;
    size_t q_rows = 0, q_width = 0;  // what the activation workspace holds
    bool q_chain_major = false;      // its Q8 blocks in chain-major order (for a chain-split GEMM only)
    hipEvent_t t0 = nullptr, t1 = nullptr;
    // decode attention scratch: scores and per-chunk maxima
    float* attn_scratch = nullptr;
    size_t cap_attn_scratch = 0;
    // one captured launch sequence (kr_capture_begin / kr_capture_end)
    bool capturing = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
};

namespace {

int fail(kr_ctx* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    return code;
}

#define HIPCHK(c, expr)                                                                            \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return fail((c), e_ == hipErrorOutOfMemory ? KR_ERR_OOM : KR_ERR_HIP, "%s: %s", #expr, \
                        hipGetErrorString(e_));                                                    \
    } while (0)

#define CHECK(c, cond, ...)                                 \
    do {                                                    \
        if (!(cond)) return fail((c), KR_ERR_INVALID, __VA_ARGS__); \
    } while (0)

DevBuf* buf_of(kr_ctx* c, kr_buf b) {
    if (b >= c->bufs.size() || !c->bufs[b].live) return nullptr;
    return &c->bufs[b];
}

Mat* mat_of(kr_ctx* c, kr_mat m) {
    if (m >= c->mats.size()) return nullptr;
    return c->mats[m];
}

#define BUF(name, handle, need)                                                                   \
    DevBuf* name = buf_of(c, handle);                                                             \
    CHECK(c, name != nullptr, "%s: unknown buffer %u", #name, (unsigned)(handle));                \
    CHECK(c, name->len >= (size_t)(need), "%s: buffer %u holds %zu elements, needs %zu", #name,   \
          (unsigned)(handle), name->len, (size_t)(need))

int ensure_workspace(kr_ctx* c, size_t rows, size_t k) {
    size_t nq = rows * k, ns = rows * (k / 32);
    if (nq > c->cap_q || ns > c->cap_s) c->epoch++;
    if (nq > c->cap_q) {
        if (c->wq) HIPCHK(c, hipFree(c->wq));
        c->wq = nullptr;
        HIPCHK(c, hipMalloc(&c->wq, nq));
        c->cap_q = nq;
    }
    if (ns > c->cap_s) {
        if (c->ws) HIPCHK(c, hipFree(c->ws));
        if (c->wh) HIPCHK(c, hipFree(c->wh));
        c->ws = nullptr;
        c->wh = nullptr;
        HIPCHK(c, hipMalloc(&c->ws, ns * sizeof(float)));
        HIPCHK(c, hipMalloc(&c->wh, ns * sizeof(uint16_t)));
        c->cap_s = ns;
    }
    return KR_OK;
}

static int ensure_workspace2(kr_ctx* c, size_t rows, size_t k) {
    const size_t nq = rows * k, ns = rows * (k / 32);
    if (nq > c->cap_q2 || ns > c->cap_s2) c->epoch++;
    if (nq > c->cap_q2) {
        if (c->wq2) HIPCHK(c, hipFree(c->wq2));
        c->wq2 = nullptr;
        HIPCHK(c, hipMalloc(&c->wq2, nq));
        c->cap_q2 = nq;
    }
    if (ns > c->cap_s2) {
        if (c->ws2) HIPCHK(c, hipFree(c->ws2));
        if (c->wh2) HIPCHK(c, hipFree(c->wh2));
        c->ws2 = nullptr;
        c->wh2 = nullptr;
        HIPCHK(c, hipMalloc(&c->ws2, ns * sizeof(float)));
        HIPCHK(c, hipMalloc(&c->wh2, ns * sizeof(uint16_t)));
        c->cap_s2 = ns;
    }
    return KR_OK;
}

int ensure_tmp(kr_ctx* c, size_t n) {
    if (n > c->cap_tmp) {
        c->epoch++;
        if (c->tmp) HIPCHK(c, hipFree(c->tmp));
        c->tmp = nullptr;
        HIPCHK(c, hipMalloc(&c->tmp, n * sizeof(float)));
        c->cap_tmp = n;
    }
    return KR_OK;
}

int stage(kr_ctx* c, IdxStage& s, const uint32_t* host, size_t n, const uint32_t** out) {
    if (s.dev && s.last.size() == n && memcmp(s.last.data(), host, n * sizeof(uint32_t)) == 0) {
        *out = s.dev;
        return KR_OK;
    }
    if (n > s.cap) {
        c->epoch++;
        if (s.dev) HIPCHK(c, hipFree(s.dev));  // hipFree waits for the device
        s.dev = nullptr;
        size_t cap = n < 256 ? 256 : n;
        HIPCHK(c, hipMalloc(&s.dev, cap * sizeof(uint32_t)));
        s.cap = cap;
    }
    if (n > s.pinned_cap) {
        for (int i = 0; i < 2; i++) {
            if (s.recorded[i]) HIPCHK(c, hipEventSynchronize(s.ev[i]));
            if (s.pinned[i]) HIPCHK(c, hipHostFree(s.pinned[i]));
            s.pinned[i] = nullptr;
            s.recorded[i] = false;
        }
        size_t cap = n < 256 ? 256 : n;
        for (int i = 0; i < 2; i++) HIPCHK(c, hipHostMalloc((void**)&s.pinned[i], cap * sizeof(uint32_t)));
        s.pinned_cap = cap;
    }
    if (!s.ev[0]) {
        HIPCHK(c, hipEventCreateWithFlags(&s.ev[0], hipEventDisableTiming));
        HIPCHK(c, hipEventCreateWithFlags(&s.ev[1], hipEventDisableTiming));
    }
    int i = s.cur ^= 1;
    if (s.recorded[i]) HIPCHK(c, hipEventSynchronize(s.ev[i]));
    memcpy(s.pinned[i], host, n * sizeof(uint32_t));
    HIPCHK(c, hipMemcpyAsync(s.dev, s.pinned[i], n * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipEventRecord(s.ev[i], c->stream));
    s.recorded[i] = true;
    s.last.assign(host, host + n);
    *out = s.dev;
    return KR_OK;
}

void free_stage(IdxStage& s) {
    for (int i = 0; i < 2; i++) {
        if (s.recorded[i]) (void)hipEventSynchronize(s.ev[i]);
        if (s.pinned[i]) (void)hipHostFree(s.pinned[i]);
        if (s.ev[i]) (void)hipEventDestroy(s.ev[i]);
    }
    if (s.dev) (void)hipFree(s.dev);
}

// (cos, sin) for positions [0, n_pos) and frequencies j < hs/2, computed with
// the reference's expressions and libm calls (cpu.rs:675-677, 697-699):
// freq = 1 / theta^((2j)/hs), angle = pos * freq, (sin, cos)(angle).
int rope_table(kr_ctx* c, float theta, size_t hs, size_t need_pos, const float2** out) {
    auto key = std::make_pair(kr::f2u(theta), hs);
    RopeTable& t = c->rope[key];
    if (t.n_pos < need_pos) {
        c->epoch++;
        size_t n_pos = need_pos;
        if (n_pos < c->seq_len) n_pos = c->seq_len;
        if (n_pos < 2 * t.n_pos) n_pos = 2 * t.n_pos;
        size_t half = hs / 2;
        std::vector<float> freq(half);
        for (size_t j = 0; j < half; j++) freq[j] = 1.0f / powf(theta, (float)(2 * j) / (float)hs);
        std::vector<float2> host(n_pos * half);
        for (size_t p = 0; p < n_pos; p++)
            for (size_t j = 0; j < half; j++) {
                float angle = (float)p * freq[j];
                host[p * half + j] = make_float2(cosf(angle), sinf(angle));
            }
        if (t.dev) HIPCHK(c, hipFree(t.dev));
        t.dev = nullptr;
        HIPCHK(c, hipMalloc(&t.dev, host.size() * sizeof(float2)));
        HIPCHK(c, hipMemcpy(t.dev, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice));
        t.n_pos = n_pos;
    }
    *out = t.dev;
    return KR_OK;
}

int new_mat(kr_ctx* c, int storage, size_t n, size_t k, kr_mat* out, Mat** mp) {
    CHECK(c, k % 32 == 0 && k > 0 && n > 0, "matrix [%zu, %zu]: in_dim must be a positive multiple of 32", n, k);
    CHECK(c, k <= 32768 && n < (1u << 31), "matrix [%zu, %zu] exceeds the supported size", n, k);
    CHECK(c, storage == KR_STORAGE_Q8_0 || storage == KR_STORAGE_Q8_0X4, "unknown storage %d", storage);
    if (storage == KR_STORAGE_Q8_0X4) CHECK(c, n % 4 == 0, "Q8_0x4 needs out_dim %% 4 == 0 (got %zu)", n);
    Mat* m = new Mat();
    m->m.storage = storage;
    m->m.n = n;
    m->m.k = k;
    size_t sbytes = n * (k / 32) * (storage == KR_STORAGE_Q8_0 ? 4 : 2);
    hipError_t e = hipMalloc(&m->m.q, n * k);
    if (e == hipSuccess) e = hipMalloc(&m->m.s, sbytes);
    if (e != hipSuccess) {
        if (m->m.q) (void)hipFree(m->m.q);
        delete m;
        return fail(c, KR_ERR_OOM, "matrix [%zu, %zu]: %s", n, k, hipGetErrorString(e));
    }
    c->mats.push_back(m);
    *out = (kr_mat)(c->mats.size() - 1);
    *mp = m;
    return KR_OK;
}

void free_devmatrix(DevMatrix& m);

// A matrix whose contents could not be produced: freed and its handle
// retired, so a failed constructor leaves nothing behind; returns rc.
int drop_new_mat(kr_ctx* c, kr_mat* out, int rc) {
    Mat* m = c->mats[*out];
    free_devmatrix(m->m);
    delete m;
    c->mats[*out] = nullptr;
    *out = KR_NO_MAT;
    return rc;
}

void free_devmatrix(DevMatrix& m) {
    if (m.q) (void)hipFree(m.q);
    if (m.s) (void)hipFree(m.s);
    m.q = nullptr;
    m.s = nullptr;
}

int sem_for_project(const DevMatrix& m) {
    return m.storage == KR_STORAGE_Q8_0X4 ? kr::SEM_FMA_CHAIN : kr::SEM_FOUR_PARTIALS_F32;
}

const Mat* proj_mat(kr_ctx* c, size_t layer, int proj) {
    if (layer >= c->proj.size() || proj < 0 || proj > 8) return nullptr;
    kr_mat m = c->proj[layer][proj];
    return m == KR_NO_MAT ? nullptr : mat_of(c, m);
}

int quantize_rows(kr_ctx* c, const float* x, size_t rows, size_t k, size_t stride) {
    int rc = ensure_workspace(c, rows, k);
    if (rc) return rc;
    HIPCHK(c, kr::launch_quantize(c->stream, x, rows, k, stride, c->wq, c->ws, c->wh));
    c->q_rows = rows;
    c->q_width = k;
    c->q_chain_major = false;
    return KR_OK;
}

kr::QuantAct act(kr_ctx* c) { return kr::QuantAct{c->wq, c->ws, c->wh}; }

// Run one or more projections that share the input x (project / project_qkv
// / project_gate_up): quantize x once, then one launch per output.
int project_many(kr_ctx* c, size_t layer, const int* projs, const kr_buf* ys, int n, kr_buf x, size_t rows) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    CHECK(c, layer < c->n_layers, "layer %zu out of range (%zu layers)", layer, c->n_layers);
    const Mat* ms[3];
    for (int i = 0; i < n; i++) {
        ms[i] = proj_mat(c, layer, projs[i]);
        CHECK(c, ms[i] != nullptr, "projection %d is not live on layer %zu", projs[i], layer);
        CHECK(c, ms[i]->m.k == ms[0]->m.k, "fused projections disagree on in_dim");
    }
    if (rows == 0) return KR_OK;
    size_t k = ms[0]->m.k;
    BUF(xb, x, rows * k);
    for (int i = 0; i < n; i++) {
        BUF(yb, ys[i], rows * ms[i]->m.n);
        (void)yb;
    }
    int rc = quantize_rows(c, xb->p, rows, k, k);
    if (rc) return rc;
    for (int i = 0; i < n; i++) {
        const DevMatrix& m = ms[i]->m;
        HIPCHK(c, kr::launch_project(c->stream, sem_for_project(m), m, act(c), rows, c->bufs[ys[i]].p, m.n, nullptr));
    }
    return KR_OK;
}

int classifier_matrix(kr_ctx* c, Mat* mt, const DevMatrix** use, int* sem) {
    if (mt->m.storage == KR_STORAGE_Q8_0) {
        *use = &mt->m;
        *sem = kr::SEM_FOUR_PARTIALS_F32;
        return KR_OK;
    }
    if (mt->requant_state < 0) {
        HIPCHK(c, hipMemsetAsync(c->counter, 0, sizeof(unsigned int), c->stream));
        HIPCHK(c, kr::launch_requant_check(c->stream, mt->m, c->counter));
        unsigned int bad = 0;
        HIPCHK(c, hipMemcpyAsync(&bad, c->counter, sizeof bad, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
        if (bad == 0) {
            mt->requant_state = 0;
        } else {
            DevMatrix& d = mt->requant;
            d.storage = KR_STORAGE_Q8_0;
            d.n = mt->m.n;
            d.k = mt->m.k;
            HIPCHK(c, hipMalloc(&d.q, d.n * d.k));
            HIPCHK(c, hipMalloc(&d.s, d.n * (d.k / 32) * sizeof(float)));
            HIPCHK(c, kr::launch_requantize(c->stream, mt->m, d));
            mt->requant_state = 1;
        }
    }
    if (mt->requant_state == 0) {
        *use = &mt->m;
        *sem = kr::SEM_FOUR_PARTIALS_F16;
    } else {
        *use = &mt->requant;
        *sem = kr::SEM_FOUR_PARTIALS_F32;
    }
    return KR_OK;
}

// The bound classifier (the embedding when tied) settles its x86 logits form
// here, at set-up: the re-quantization check reads a counter back, and doing
// it inside the first logits() would make that call a host barrier.
int prime_classifier(kr_ctx* c) {
    Mat* mt = mat_of(c, c->classifier == KR_NO_MAT ? c->embedding : c->classifier);
    if (!mt) return KR_OK;
    const DevMatrix* m;
    int sem;
    return classifier_matrix(c, mt, &m, &sem);
}

int logits_with(kr_ctx* c, Mat* mt, kr_buf x, kr_buf y) {
    const DevMatrix* m;
    int sem;
    int rc = classifier_matrix(c, mt, &m, &sem);
    if (rc) return rc;
    BUF(xb, x, m->k);
    BUF(yb, y, m->n);
    rc = quantize_rows(c, xb->p, 1, m->k, m->k);
    if (rc) return rc;
    HIPCHK(c, kr::launch_project(c->stream, sem, *m, act(c), 1, yb->p, m->n, nullptr));
    return KR_OK;
}

std::vector<uint32_t> to_u32(const size_t* v, size_t n) {
    std::vector<uint32_t> out(n);
    for (size_t i = 0; i < n; i++) out[i] = (uint32_t)v[i];
    return out;
}

// The chain-split prefill GEMM applies to a Q8_0 matrix with K % 128 == 0
// (four equal partial sums) and few rows, where the plain tiles leave most of
// the device idle, and where its own grid (64x64 tiles x 4 partial sums) still
// has a workgroup for every CU (at 64 rows of a 1024-wide output it has 64,
// and the plain 32x32 tiles are faster).
bool chain_split_ok(const DevMatrix& m, size_t rows) {
    return m.storage == KR_STORAGE_Q8_0 && m.k % 128 == 0 && rows >= 8 && rows <= 256 &&
           ((rows + 63) / 64) * ((m.n + 63) / 64) * 4 >= 256;
}

int ensure_chain_major(kr_ctx* c, const Mat* mt, const DevMatrix** out) {
    Mat* m = const_cast<Mat*>(mt);
    if (!m->cm.q) {
        DevMatrix cm{};
        cm.storage = KR_STORAGE_Q8_0, cm.n = m->m.n, cm.k = m->m.k;
        hipError_t e = hipMalloc(&cm.q, cm.n * cm.k);
        if (e == hipSuccess) e = hipMalloc(&cm.s, cm.n * (cm.k / 32) * sizeof(float));
        if (e == hipSuccess) e = kr::launch_chain_major(c->stream, m->m, cm.q, (float*)cm.s);
        if (e != hipSuccess) {
            free_devmatrix(cm);
            HIPCHK(c, e);
        }
        m->cm = cm;
    }
    *out = &m->cm;
    return KR_OK;
}

}  // namespace

extern "C" {

int kr_open(int device, kr_ctx** out, char* detail, size_t detail_len) {
    auto say = [&](const char* msg) {
        if (detail && detail_len) snprintf(detail, detail_len, "%s", msg);
    };
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) {
        say("no HIP device on this machine");
        return KR_ERR_NO_DEVICE;
    }
    if (device < 0 || device >= count) {
        say("no HIP device with that index");
        return KR_ERR_NO_DEVICE;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        say("no HIP device: properties query failed");
        return KR_ERR_NO_DEVICE;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        char msg[256];
        snprintf(msg, sizeof msg, "no gfx950 HIP device (device %d is %s)", device, prop.gcnArchName);
        say(msg);
        return KR_ERR_NO_DEVICE;
    }
    kr_ctx* c = new kr_ctx();
    c->device = device;
    c->devname = prop.name[0] ? prop.name : prop.gcnArchName;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc(&c->tokens, kr_ctx::kTokens * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&c->counter, sizeof(unsigned int)) != hipSuccess ||
        hipMemset(c->tokens, 0, kr_ctx::kTokens * sizeof(uint32_t)) != hipSuccess ||
        scratch_address(device, &c->scratch) != hipSuccess) {
        say("HIP device present but failed to start");
        kr_close(c);
        return KR_ERR_HIP;
    }
    *out = c;
    return KR_OK;
}

void kr_close(kr_ctx* c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (DevBuf& b : c->bufs)
        if (b.p) (void)hipFree(b.p);
    for (Mat* m : c->mats)
        if (m) {
            free_devmatrix(m->m);
            free_devmatrix(m->requant);
            free_devmatrix(m->cm);
            delete m;
        }
    for (auto& kv : c->rope)
        if (kv.second.dev) (void)hipFree(kv.second.dev);
    free_stage(c->st_pos);
    free_stage(c->st_slots);
    free_stage(c->st_win);
    free_stage(c->st_tok);
    void* ptrs[] = {c->kc, c->vc, c->wq, c->ws, c->wh, c->wq2, c->ws2, c->wh2, c->tmp, c->tokens, c->counter,
                    c->attn_scratch};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    if (c->t0) (void)hipEventDestroy(c->t0);
    if (c->t1) (void)hipEventDestroy(c->t1);
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char* kr_last_error(const kr_ctx* c) { return c ? c->err.c_str() : "no context"; }
const char* kr_name(const kr_ctx*) { return "hip"; }
const char* kr_storage(const kr_ctx* c) { return c->storage; }

int kr_device_name(const kr_ctx* c, char* out, size_t len) {
    snprintf(out, len, "%s", c->devname.c_str());
    return KR_OK;
}

int kr_matrix_q8_0(kr_ctx* c, size_t n, size_t k, const int8_t* quants, const float* scales, kr_mat* out) {
    Mat* m;
    int rc = new_mat(c, KR_STORAGE_Q8_0, n, k, out, &m);
    if (rc) return rc;
    hipError_t e = hipMemcpy(m->m.q, quants, n * k, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(m->m.s, scales, n * (k / 32) * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess)
        return drop_new_mat(c, out, fail(c, KR_ERR_HIP, "uploading matrix [%zu, %zu]: %s", n, k, hipGetErrorString(e)));
    return KR_OK;
}

// De-interleave Q8Block4 groups (quant.rs:113-118, layout quant.rs:147-153)
// into row-major quants and per-row f16 scale bits; the inverse of
// Q8_0x4::from_f32's packing, lossless like to_row_major (quant.rs:198-219).
int kr_matrix_q8_0x4(kr_ctx* c, size_t n, size_t k, const void* blocks, kr_mat* out) {
    Mat* m;
    int rc = new_mat(c, KR_STORAGE_Q8_0X4, n, k, out, &m);
    if (rc) return rc;
    size_t nb = k / 32;
    std::vector<int8_t> q(n * k);
    std::vector<uint16_t> s(n * nb);
    const uint8_t* src = (const uint8_t*)blocks;
    for (size_t g = 0; g < n / 4; g++)
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = src + (g * nb + b) * 136;
            uint16_t sc[4];
            memcpy(sc, blk, 8);
            const int8_t* qs = (const int8_t*)(blk + 8);
            for (size_t r = 0; r < 4; r++) {
                size_t row = g * 4 + r;
                s[row * nb + b] = sc[r];
                int8_t* dst = &q[row * k + b * 32];
                for (size_t seg = 0; seg < 8; seg++)
                    for (size_t lane = 0; lane < 4; lane++) dst[seg * 4 + lane] = qs[seg * 16 + r * 4 + lane];
            }
        }
    hipError_t e = hipMemcpy(m->m.q, q.data(), q.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(m->m.s, s.data(), s.size() * sizeof(uint16_t), hipMemcpyHostToDevice);
    if (e != hipSuccess)
        return drop_new_mat(c, out, fail(c, KR_ERR_HIP, "uploading matrix [%zu, %zu]: %s", n, k, hipGetErrorString(e)));
    return KR_OK;
}

int kr_matrix_quantize(kr_ctx* c, int storage, int src_kind, const void* data, size_t n, size_t k, kr_mat* out) {
    CHECK(c, src_kind == KR_SRC_F32 || src_kind == KR_SRC_BF16, "unknown source kind %d", src_kind);
    CHECK(c, data != nullptr, "no source data");
    Mat* m;
    int rc = new_mat(c, storage, n, k, out, &m);
    if (rc) return rc;
    // rows go through a device staging buffer in chunks of about 64 MiB
    const size_t esz = src_kind == KR_SRC_F32 ? 4 : 2, row_bytes = k * esz;
    const size_t chunk = std::max<size_t>(1, (64u << 20) / row_bytes);
    void* stage_dev = nullptr;
    hipError_t e0 = hipStreamSynchronize(c->stream);
    if (e0 == hipSuccess) e0 = hipMalloc(&stage_dev, std::min(chunk, n) * row_bytes);
    if (e0 != hipSuccess)
        return drop_new_mat(c, out, fail(c, e0 == hipErrorOutOfMemory ? KR_ERR_OOM : KR_ERR_HIP,
                                         "staging matrix [%zu, %zu]: %s", n, k, hipGetErrorString(e0)));
    int err = KR_OK;
    for (size_t r0 = 0; r0 < n && err == KR_OK; r0 += chunk) {
        const size_t rows = std::min(chunk, n - r0);
        hipError_t e = hipMemcpy(stage_dev, (const uint8_t*)data + r0 * row_bytes, rows * row_bytes,
                                 hipMemcpyHostToDevice);
        if (e == hipSuccess) e = kr::launch_quant_weights(c->stream, m->m, r0, rows, stage_dev, src_kind == KR_SRC_BF16);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);  // the next chunk reuses the staging buffer
        if (e != hipSuccess) err = fail(c, KR_ERR_HIP, "quantizing matrix [%zu, %zu]: %s", n, k, hipGetErrorString(e));
    }
    (void)hipFree(stage_dev);
    return err == KR_OK ? KR_OK : drop_new_mat(c, out, err);
}

int kr_matrix_synthetic(kr_ctx* c, int storage, size_t n, size_t k, uint64_t seed, float stddev, kr_mat* out) {
    Mat* m;
    int rc = new_mat(c, storage, n, k, out, &m);
    if (rc) return rc;
    hipError_t e = kr::launch_synthetic_q8(c->stream, m->m, seed, stddev);
    if (e != hipSuccess)
        return drop_new_mat(c, out, fail(c, KR_ERR_HIP, "synthetic matrix [%zu, %zu]: %s", n, k, hipGetErrorString(e)));
    return KR_OK;
}

// workgroups x rounds of kr_mfma_rate: 2^32 is ~0.6 s of 32x32x32 int8 MFMAs
static constexpr uint64_t kMfmaProbeMax = 1ull << 32;

int kr_mfma_rate(kr_ctx* c, int kind, size_t workgroups, size_t iters, double* ops) {
    CHECK(c, kind == 0 || kind == 1, "MFMA kind %d", kind);
    CHECK(c, workgroups > 0 && workgroups <= (1u << 20) && iters > 0 && iters < (1u << 31), "probe size");
    // about a second of MFMA work at the chip's rate at most: a longer probe
    // would hold the GPU like a hang
    CHECK(c, (double)workgroups * (double)iters <= (double)kMfmaProbeMax,
          "probe of %zu workgroups x %zu rounds exceeds the %llu limit", workgroups, iters,
          (unsigned long long)kMfmaProbeMax);
    int rc = ensure_tmp(c, workgroups * 256);
    if (rc) return rc;
    HIPCHK(c, kr::launch_mfma_spin(c->stream, kind, (int*)c->tmp, workgroups, (uint32_t)iters, ops));
    return KR_OK;
}

int kr_synthetic_values(kr_ctx* c, kr_buf out, size_t n, uint64_t seed, float stddev) {
    BUF(ob, out, n);
    HIPCHK(c, kr::launch_synthetic_values(c->stream, ob->p, n, seed, stddev));
    return KR_OK;
}

int kr_matrix_free(kr_ctx* c, kr_mat h) {
    Mat* m = mat_of(c, h);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)h);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    free_devmatrix(m->m);
    free_devmatrix(m->requant);
    free_devmatrix(m->cm);
    delete m;
    c->mats[h] = nullptr;
    return KR_OK;
}

int kr_bind_embedding(kr_ctx* c, kr_mat m) {
    CHECK(c, mat_of(c, m) != nullptr, "unknown matrix %u", (unsigned)m);
    c->embedding = m;
    return c->prepared ? prime_classifier(c) : KR_OK;
}

int kr_bind_classifier(kr_ctx* c, kr_mat m) {
    CHECK(c, m == KR_NO_MAT || mat_of(c, m) != nullptr, "unknown matrix %u", (unsigned)m);
    c->classifier = m;
    return c->prepared ? prime_classifier(c) : KR_OK;
}

int kr_bind_proj(kr_ctx* c, size_t layer, int proj, kr_mat m) {
    CHECK(c, proj >= 0 && proj <= 8, "projection index %d out of range", proj);
    CHECK(c, m == KR_NO_MAT || mat_of(c, m) != nullptr, "unknown matrix %u", (unsigned)m);
    if (c->proj.size() <= layer) {
        std::array<kr_mat, 9> none;
        none.fill(KR_NO_MAT);
        c->proj.resize(layer + 1, none);
    }
    c->proj[layer][proj] = m;
    return KR_OK;
}

int kr_prepare(kr_ctx* c, size_t n_layers, size_t kv_dim, size_t seq_len) {
    CHECK(c, !c->prepared, "prepare() is called once");
    Mat* e = mat_of(c, c->embedding);
    CHECK(c, e != nullptr, "prepare() needs an embedding matrix bound");
    HIPCHK(c, hipSetDevice(c->device));
    if (c->proj.size() < n_layers) {
        std::array<kr_mat, 9> none;
        none.fill(KR_NO_MAT);
        c->proj.resize(n_layers, none);
    }
    size_t n = n_layers * seq_len * kv_dim;
    if (n) {
        HIPCHK(c, hipMalloc(&c->kc, n * sizeof(float)));
        HIPCHK(c, hipMalloc(&c->vc, n * sizeof(float)));
        HIPCHK(c, hipMemsetAsync(c->kc, 0, n * sizeof(float), c->stream));
        HIPCHK(c, hipMemsetAsync(c->vc, 0, n * sizeof(float), c->stream));
    }
    c->n_layers = n_layers;
    c->kv_dim = kv_dim;
    c->seq_len = seq_len;
    c->storage = e->m.storage == KR_STORAGE_Q8_0 ? "q8_0" : "q8_0x4";
    c->prepared = true;
    return prime_classifier(c);
}

int kr_alloc(kr_ctx* c, size_t len, kr_buf* out) {
    DevBuf b;
    b.len = len;
    b.live = true;
    if (len) {
        HIPCHK(c, hipMalloc(&b.p, len * sizeof(float)));
        HIPCHK(c, hipMemsetAsync(b.p, 0, len * sizeof(float), c->stream));
    }
    c->bufs.push_back(b);
    *out = (kr_buf)(c->bufs.size() - 1);
    return KR_OK;
}

int kr_upload(kr_ctx* c, const float* data, size_t len, kr_buf* out) {
    DevBuf b;
    b.len = len;
    b.live = true;
    if (len) {
        HIPCHK(c, hipMalloc(&b.p, len * sizeof(float)));
        HIPCHK(c, hipMemcpyAsync(b.p, data, len * sizeof(float), hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
    }
    c->bufs.push_back(b);
    *out = (kr_buf)(c->bufs.size() - 1);
    return KR_OK;
}

int kr_read(kr_ctx* c, kr_buf src, float* out, size_t len) {
    BUF(s, src, len);
    if (len) HIPCHK(c, hipMemcpyAsync(out, s->p, len * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_embed(kr_ctx* c, size_t token, kr_buf out, size_t offset) {
    Mat* e = mat_of(c, c->embedding);
    CHECK(c, c->prepared && e != nullptr, "prepare() runs before any compute");
    CHECK(c, token < e->m.n, "token %zu out of range (vocab %zu)", token, e->m.n);
    BUF(o, out, offset + e->m.k);
    HIPCHK(c, kr::launch_embed(c->stream, e->m, token, nullptr, o->p + offset));
    return KR_OK;
}

int kr_copy(kr_ctx* c, kr_buf src, size_t so, kr_buf dst, size_t doff, size_t len) {
    BUF(s, src, so + len);
    BUF(d, dst, doff + len);
    if (len == 0) return KR_OK;
    bool overlap = src == dst && so < doff + len && doff < so + len && so != doff;
    if (so == doff && src == dst) return KR_OK;
    if (overlap) {  // memmove semantics (cpu.rs:230-232)
        int rc = ensure_tmp(c, len);
        if (rc) return rc;
        HIPCHK(c, kr::launch_copy(c->stream, c->tmp, s->p + so, len));
        HIPCHK(c, kr::launch_copy(c->stream, d->p + doff, c->tmp, len));
        return KR_OK;
    }
    HIPCHK(c, kr::launch_copy(c->stream, d->p + doff, s->p + so, len));
    return KR_OK;
}

int kr_rms_norm(kr_ctx* c, kr_buf out, kr_buf x, kr_buf w, size_t rows, size_t dim, float eps) {
    BUF(o, out, rows * dim);
    BUF(xb, x, rows * dim);
    BUF(wb, w, dim);
    CHECK(c, dim <= 16000, "rms_norm dim %zu exceeds 16000", dim);  // LDS holds dim squares
    HIPCHK(c, kr::launch_rms_norm(c->stream, o->p, xb->p, wb->p, rows, dim, eps));
    return KR_OK;
}

int kr_qk_norm(kr_ctx* c, kr_buf v, size_t rows, size_t width, size_t head, kr_buf w, float eps) {
    CHECK(c, head > 0 && head <= 256, "head_size must be in 1..=256");
    BUF(vb, v, rows * width);
    BUF(wb, w, head);
    HIPCHK(c, kr::launch_qk_norm(c->stream, vb->p, rows, width, head, wb->p, eps));
    return KR_OK;
}

int kr_rope(kr_ctx* c, kr_buf q, kr_buf k, size_t qw, size_t kvw, size_t rows, const size_t* positions,
            const kr_rope_spec* spec) {
    CHECK(c, spec && spec->head_size >= 2 && spec->head_size % 2 == 0, "rope head_size must be even");
    BUF(qb, q, rows * qw);
    BUF(kb, k, rows * kvw);
    if (rows == 0) return KR_OK;
    size_t maxp = 0;
    for (size_t i = 0; i < rows; i++) maxp = positions[i] > maxp ? positions[i] : maxp;
    CHECK(c, maxp < (1u << 24), "rope position %zu too large", maxp);
    const float2* tab;
    int rc = rope_table(c, spec->theta, spec->head_size, maxp + 1, &tab);
    if (rc) return rc;
    std::vector<uint32_t> p = to_u32(positions, rows);
    const uint32_t* pd;
    rc = stage(c, c->st_pos, p.data(), rows, &pd);
    if (rc) return rc;
    HIPCHK(c, kr::launch_rope(c->stream, qb->p, kb->p, qw, kvw, rows, pd, tab, spec->head_size, spec->interleaved));
    return KR_OK;
}

int kr_project(kr_ctx* c, size_t layer, int proj, kr_buf x, kr_buf y, size_t rows) {
    return project_many(c, layer, &proj, &y, 1, x, rows);
}

int kr_project_qkv(kr_ctx* c, size_t layer, kr_buf x, kr_buf q, kr_buf k, kr_buf v, size_t rows) {
    int projs[3] = {KR_PROJ_Q, KR_PROJ_K, KR_PROJ_V};
    kr_buf ys[3] = {q, k, v};
    return project_many(c, layer, projs, ys, 3, x, rows);
}

int kr_project_gate_up(kr_ctx* c, size_t layer, kr_buf x, kr_buf gate, kr_buf up, size_t rows) {
    int projs[2] = {KR_PROJ_GATE, KR_PROJ_UP};
    kr_buf ys[2] = {gate, up};
    return project_many(c, layer, projs, ys, 2, x, rows);
}

int kr_kv_write(kr_ctx* c, size_t layer, const size_t* slots, kr_buf k, kr_buf v, size_t rows) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    CHECK(c, layer < c->n_layers, "layer %zu out of range", layer);
    BUF(kb, k, rows * c->kv_dim);
    BUF(vb, v, rows * c->kv_dim);
    if (rows == 0) return KR_OK;
    for (size_t i = 0; i < rows; i++) CHECK(c, slots[i] < c->seq_len, "slot %zu out of range", slots[i]);
    std::vector<uint32_t> s = to_u32(slots, rows);
    const uint32_t* sd;
    int rc = stage(c, c->st_slots, s.data(), rows, &sd);
    if (rc) return rc;
    HIPCHK(c, kr::launch_kv_write(c->stream, c->kc, c->vc, layer, c->seq_len, c->kv_dim, sd, kb->p, vb->p, rows));
    return KR_OK;
}

// The split-attention scratch (scores and chunk maxima), grown on demand.
int ensure_attn_scratch(kr_ctx* c, size_t need) {
    if (need > c->cap_attn_scratch) {
        if (c->attn_scratch) HIPCHK(c, hipFree(c->attn_scratch));  // hipFree waits for the device
        c->attn_scratch = nullptr;
        HIPCHK(c, hipMalloc(&c->attn_scratch, need * sizeof(float)));
        c->cap_attn_scratch = need;
        c->epoch++;
    }
    return KR_OK;
}

// Attention over n >= 1 rows with host windows `w` (staged at `wd`): rows
// whose windows differ (batched decode of separate sequences) take the
// two-launch split form, everything else launch_attention.
int attention_many(kr_ctx* c, const float* q, float* out, float* att, size_t layer, const uint32_t* wd,
                   const std::vector<uint32_t>& w, size_t n, size_t max_count, const kr_attn_spec* sp,
                   int8_t* qo, float* so, uint16_t* ho, bool keep_att = true) {
    const kr::DevWindow* hw = (const kr::DevWindow*)w.data();
    const float scale = 1.0f / sqrtf((float)sp->head_size);  // cpu.rs:591
    if (n >= 2 && !kr::attention_rows_uniform(hw, n, max_count, sp->kv_mul, sp->head_size) &&
        kr::attention_split_rows_ok(max_count, sp->kv_mul, sp->head_size)) {
        int rc = ensure_attn_scratch(c, n * kr::attention_split_scratch(sp->n_heads, c->seq_len));
        if (rc) return rc;
        HIPCHK(c, kr::launch_attention_split_rows(c->stream, q, out, att, c->kc, c->vc, layer, (const kr::DevWindow*)wd,
                                                  n, max_count, sp->n_heads, sp->kv_mul, sp->head_size, sp->kv_dim,
                                                  sp->seq_len, scale, c->attn_scratch, keep_att,
                                                  sp->head_size % 32 == 0 ? qo : nullptr, so, ho));
        const size_t width = sp->n_heads * sp->head_size;
        if (qo && sp->head_size % 32 != 0) HIPCHK(c, kr::launch_quantize(c->stream, out, n, width, width, qo, so, ho));
        return KR_OK;
    }
    // the matrix-core prefill attention keeps each pair's max and sum in the scratch
    int rc = ensure_attn_scratch(c, 2 * n * sp->n_heads);
    if (rc) return rc;
    HIPCHK(c, kr::launch_attention(c->stream, q, out, att, c->kc, c->vc, layer, (const kr::DevWindow*)wd, n, max_count,
                                   sp->n_heads, sp->kv_mul, sp->head_size, sp->kv_dim, sp->seq_len, scale, qo, so, ho,
                                   hw, c->attn_scratch, keep_att));
    return KR_OK;
}

int kr_attention(kr_ctx* c, kr_buf q, kr_buf out, kr_buf att, size_t layer, const kr_window* windows,
                 size_t n, const kr_attn_spec* sp) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    CHECK(c, layer < c->n_layers, "layer %zu out of range", layer);
    CHECK(c, sp && sp->kv_dim == c->kv_dim && sp->seq_len == c->seq_len,
          "attention spec does not match the prepared cache");
    CHECK(c, sp->head_size % 4 == 0 && sp->head_size <= 256, "head_size must be a multiple of 4, at most 256");
    CHECK(c, sp->head_size > 0 && sp->kv_mul > 0 && sp->n_heads % sp->kv_mul == 0 &&
                 (sp->n_heads / sp->kv_mul) * sp->head_size <= sp->kv_dim,
          "attention geometry is inconsistent");
    size_t width = sp->n_heads * sp->head_size;
    BUF(qb, q, n * width);
    BUF(ob, out, n * width);
    BUF(ab, att, n * sp->n_heads * sp->seq_len);
    if (n == 0) return KR_OK;
    std::vector<uint32_t> w(4 * n);
    size_t max_count = 0;
    for (size_t i = 0; i < n; i++) {
        const kr_window& x = windows[i];
        CHECK(c, x.att_start <= x.slot && x.slot < c->seq_len && x.shared_start <= x.shared_end &&
                     x.shared_end <= c->seq_len,
              "window %zu out of range", i);
        size_t count = (x.shared_end - x.shared_start) + x.slot - x.att_start + 1;
        CHECK(c, count <= c->seq_len, "window %zu attends more than seq_len slots", i);
        max_count = count > max_count ? count : max_count;
        w[4 * i] = (uint32_t)x.att_start;
        w[4 * i + 1] = (uint32_t)x.slot;
        w[4 * i + 2] = (uint32_t)x.shared_start;
        w[4 * i + 3] = (uint32_t)x.shared_end;
    }
    const uint32_t* wd;
    int rc = stage(c, c->st_win, w.data(), 4 * n, &wd);
    if (rc) return rc;
    return attention_many(c, qb->p, ob->p, ab->p, layer, wd, w, n, max_count, sp, nullptr, nullptr, nullptr);
}

int kr_add_in_place(kr_ctx* c, kr_buf dst, kr_buf src, size_t len) {
    BUF(d, dst, len);
    BUF(s, src, len);
    HIPCHK(c, kr::launch_add(c->stream, d->p, s->p, len));
    return KR_OK;
}

int kr_mul(kr_ctx* c, kr_buf out, size_t oo, kr_buf a, size_t ao, kr_buf b, size_t bo, size_t len) {
    BUF(o, out, oo + len);
    BUF(ab, a, ao + len);
    BUF(bb, b, bo + len);
    auto hazard = [&](kr_buf in, size_t io) {
        return in == out && io != oo && io < oo + len && oo < io + len;
    };
    int seq = hazard(a, ao) || hazard(b, bo);
    HIPCHK(c, kr::launch_mul(c->stream, o->p + oo, ab->p + ao, bb->p + bo, len, seq));
    return KR_OK;
}

int kr_conv_prefill(kr_ctx* c, kr_buf out, kr_buf x, kr_buf kernel, size_t rows, size_t dim, size_t k) {
    CHECK(c, k >= 1, "conv kernel width must be positive");
    BUF(o, out, rows * dim);
    BUF(xb, x, rows * dim);
    BUF(kb, kernel, dim * k);
    CHECK(c, out != x, "conv_prefill output must not alias its input");
    HIPCHK(c, kr::launch_conv_prefill(c->stream, o->p, xb->p, kb->p, rows, dim, k));
    return KR_OK;
}

int kr_conv_decode(kr_ctx* c, kr_buf out, kr_buf x, kr_buf kernel, kr_buf state, size_t dim, size_t k) {
    CHECK(c, k >= 1, "conv kernel width must be positive");
    BUF(o, out, dim);
    BUF(xb, x, dim);
    BUF(kb, kernel, dim * k);
    BUF(sb, state, (k - 1) * dim);
    HIPCHK(c, kr::launch_conv_decode(c->stream, o->p, xb->p, kb->p, sb->p, dim, k));
    return KR_OK;
}

int kr_silu_mul(kr_ctx* c, kr_buf gate, kr_buf up, size_t len) {
    BUF(g, gate, len);
    BUF(u, up, len);
    HIPCHK(c, kr::launch_silu_mul(c->stream, g->p, u->p, len));
    return KR_OK;
}

int kr_logits(kr_ctx* c, kr_buf x, kr_buf y) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    Mat* m = mat_of(c, c->classifier != KR_NO_MAT ? c->classifier : c->embedding);
    CHECK(c, m != nullptr, "no classifier bound");
    return logits_with(c, m, x, y);
}

int kr_matmul(kr_ctx* c, kr_mat w, kr_buf x, kr_buf y, size_t rows) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    BUF(xb, x, rows * m->m.k);
    BUF(yb, y, rows * m->m.n);
    if (rows == 0) return KR_OK;
    int rc = quantize_rows(c, xb->p, rows, m->m.k, m->m.k);
    if (rc) return rc;
    HIPCHK(c, kr::launch_project(c->stream, sem_for_project(m->m), m->m, act(c), rows, yb->p, m->m.n, nullptr));
    return KR_OK;
}

// kr_matmul with the activation quantization in this device's `scratch`
// array: no hipMalloc, hipFree or other allocating call. The context's own
// workspace (what kr_matmul_quantized reads) is left untouched.
int kr_matmul_noalloc(kr_ctx* c, kr_mat w, kr_buf x, kr_buf y, size_t rows) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    BUF(xb, x, rows * m->m.k);
    BUF(yb, y, rows * m->m.n);
    CHECK(c, rows <= kNoAllocMaxElems / m->m.k, "rows * in_dim = %zu * %zu exceeds the no-allocation limit of %zu",
          rows, m->m.k, kNoAllocMaxElems);
    CHECK(c, c->scratch != nullptr, "no scratch array on this device");
    if (rows == 0) return KR_OK;
    int8_t* q = (int8_t*)c->scratch;
    float* s = (float*)(c->scratch + kScratchQuants);
    uint16_t* h = (uint16_t*)(c->scratch + kScratchQuants + kScratchScales);
    HIPCHK(c, kr::launch_quantize(c->stream, xb->p, rows, m->m.k, m->m.k, q, s, h));
    HIPCHK(c, kr::launch_project(c->stream, sem_for_project(m->m), m->m, kr::QuantAct{q, s, h}, rows, yb->p, m->m.n,
                                 nullptr));
    return KR_OK;
}

size_t kr_matmul_noalloc_max_elems(void) { return kNoAllocMaxElems; }

int kr_quantize_rows(kr_ctx* c, kr_buf x, size_t rows, size_t width) {
    CHECK(c, width % 32 == 0 && width > 0, "width must be a positive multiple of 32");
    BUF(xb, x, rows * width);
    return quantize_rows(c, xb->p, rows, width, width);
}

int kr_matmul_quantized(kr_ctx* c, kr_mat w, kr_buf y, size_t rows) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    CHECK(c, rows <= c->q_rows && m->m.k == c->q_width && !c->q_chain_major,
          "the workspace holds %zu rows of %zu, not %zu of %zu", c->q_rows, c->q_width, rows, m->m.k);
    BUF(yb, y, rows * m->m.n);
    if (rows == 0) return KR_OK;
    HIPCHK(c, kr::launch_project(c->stream, sem_for_project(m->m), m->m, act(c), rows, yb->p, m->m.n, nullptr));
    return KR_OK;
}

int kr_matmul_split(kr_ctx* c, kr_mat w, kr_buf x, kr_buf y, size_t rows) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    CHECK(c, m->m.storage == KR_STORAGE_Q8_0 && m->m.k % 128 == 0,
          "the chain-split projection needs a Q8_0 matrix with in_dim %% 128 == 0");
    BUF(yb, y, 4 * rows * m->m.n);
    if (x != KR_NO_BUF) {
        BUF(xb, x, rows * m->m.k);
        int rc = ensure_workspace(c, rows, m->m.k);
        if (rc) return rc;
        HIPCHK(c, kr::launch_quantize(c->stream, xb->p, rows, m->m.k, m->m.k, c->wq, c->ws, c->wh, true));
        c->q_rows = rows;
        c->q_width = m->m.k;
        c->q_chain_major = true;
    }
    CHECK(c, rows <= c->q_rows && m->m.k == c->q_width && c->q_chain_major,
          "the workspace does not hold %zu chain-major rows of %zu", rows, m->m.k);
    if (rows == 0) return KR_OK;
    const DevMatrix* cm = nullptr;
    int rc = ensure_chain_major(c, m, &cm);
    if (rc) return rc;
    HIPCHK(c, kr::launch_gemm_q8_cs(c->stream, *cm, act(c), rows, yb->p));
    return KR_OK;
}

int kr_matmul_quantized_set(kr_ctx* c, const kr_mat* w, const kr_buf* y, int n, size_t rows) {
    CHECK(c, n >= 1 && n <= 3 && w && y, "1 to 3 matrices per launch");
    const DevMatrix* ms[3];
    float* yp[3];
    for (int i = 0; i < n; i++) {
        Mat* m = mat_of(c, w[i]);
        CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w[i]);
        ms[i] = &m->m;
        CHECK(c, rows <= c->q_rows && ms[i]->k == c->q_width && !c->q_chain_major,
              "the workspace holds %zu rows of %zu, not %zu of %zu", c->q_rows, c->q_width, rows, ms[i]->k);
        CHECK(c, ms[i]->storage == ms[0]->storage, "the matrices of one launch share their storage");
        BUF(yb, y[i], rows * ms[i]->n);
        yp[i] = yb->p;
    }
    if (rows == 0) return KR_OK;
    HIPCHK(c, kr::launch_project_set(c->stream, sem_for_project(*ms[0]), ms, yp, n, act(c), rows, nullptr));
    return KR_OK;
}

int kr_stream_read(kr_ctx* c, kr_buf src, size_t offset, size_t len) {
    return kr_stream_read_shape(c, src, offset, len, 2, 0);
}

int kr_stream_read_shape(kr_ctx* c, kr_buf src, size_t offset, size_t len, int chunks_per_lane,
                         size_t workgroups) {
    BUF(s, src, offset + len);
    CHECK(c, offset % 4 == 0 && len % 4 == 0, "offset and length are multiples of 4 floats");
    CHECK(c, chunks_per_lane == 1 || chunks_per_lane == 2 || chunks_per_lane == 4 || chunks_per_lane == 8,
          "chunks per lane %d (1, 2, 4 or 8)", chunks_per_lane);
    CHECK(c, workgroups <= (1u << 20), "workgroups %zu", workgroups);
    HIPCHK(c, kr::launch_stream_read(c->stream, s->p + offset, len, (int*)c->counter, chunks_per_lane, workgroups));
    return KR_OK;
}

int kr_capture_begin(kr_ctx* c) {
    CHECK(c, !c->capturing, "a capture is already open");
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->graph_exec = nullptr;
    c->graph = nullptr;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    return KR_OK;
}

int kr_capture_end(kr_ctx* c) {
    CHECK(c, c->capturing, "no capture is open");
    c->capturing = false;
    HIPCHK(c, hipStreamEndCapture(c->stream, &c->graph));
    HIPCHK(c, hipGraphInstantiate(&c->graph_exec, c->graph, nullptr, nullptr, 0));
    return KR_OK;
}

int kr_replay(kr_ctx* c, size_t times) {
    CHECK(c, c->graph_exec != nullptr, "nothing was captured");
    for (size_t i = 0; i < times; i++) HIPCHK(c, hipGraphLaunch(c->graph_exec, c->stream));
    return KR_OK;
}

int kr_timer_start(kr_ctx* c) {
    if (!c->t0) {
        HIPCHK(c, hipEventCreate(&c->t0));
        HIPCHK(c, hipEventCreate(&c->t1));
    }
    HIPCHK(c, hipEventRecord(c->t0, c->stream));
    return KR_OK;
}

int kr_timer_stop(kr_ctx* c, float* ms) {
    CHECK(c, c->t0 != nullptr, "kr_timer_start was not called");
    HIPCHK(c, hipEventRecord(c->t1, c->stream));
    HIPCHK(c, hipEventSynchronize(c->t1));
    HIPCHK(c, hipEventElapsedTime(ms, c->t0, c->t1));
    return KR_OK;
}

int kr_classify(kr_ctx* c, kr_mat w, kr_buf x, kr_buf y) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    return logits_with(c, m, x, y);
}

int kr_dbg_quantize(kr_ctx* c, kr_buf x, size_t rows, size_t width, int8_t* quants, float* scales,
                    uint16_t* scales_f16) {
    CHECK(c, width % 32 == 0 && width > 0, "width must be a positive multiple of 32");
    BUF(xb, x, rows * width);
    int rc = quantize_rows(c, xb->p, rows, width, width);
    if (rc) return rc;
    size_t nb = rows * width / 32;
    HIPCHK(c, hipMemcpyAsync(quants, c->wq, rows * width, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(scales, c->ws, nb * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(scales_f16, c->wh, nb * sizeof(uint16_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_dbg_block_dots(kr_ctx* c, kr_mat w, kr_buf x, size_t rows, int32_t* out) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    BUF(xb, x, rows * m->m.k);
    if (rows == 0) return KR_OK;
    size_t n = rows * m->m.n * (m->m.k / 32);
    int32_t* d = nullptr;
    float* y = nullptr;
    HIPCHK(c, hipMalloc(&d, n * sizeof(int32_t)));
    HIPCHK(c, hipMalloc(&y, rows * m->m.n * sizeof(float)));
    int rc = quantize_rows(c, xb->p, rows, m->m.k, m->m.k);
    if (rc == KR_OK) {
        hipError_t e = kr::launch_project(c->stream, sem_for_project(m->m), m->m, act(c), rows, y, m->m.n, d);
        if (e == hipSuccess) e = hipMemcpyAsync(out, d, n * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = fail(c, KR_ERR_HIP, "block dots: %s", hipGetErrorString(e));
    }
    (void)hipFree(d);
    (void)hipFree(y);
    return rc;
}

int kr_kv_upload(kr_ctx* c, int which, size_t offset, const float* data, size_t len) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    CHECK(c, offset + len <= c->n_layers * c->seq_len * c->kv_dim, "cache range out of bounds");
    float* base = which == 0 ? c->kc : c->vc;
    HIPCHK(c, hipMemcpyAsync(base + offset, data, len * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_kv_read(kr_ctx* c, int which, size_t offset, float* out, size_t len) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    CHECK(c, offset + len <= c->n_layers * c->seq_len * c->kv_dim, "cache range out of bounds");
    const float* base = which == 0 ? c->kc : c->vc;
    HIPCHK(c, hipMemcpyAsync(out, base + offset, len * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_dbg_mfma_f32(kr_ctx* c, const float* a, const float* b, const float* acc, float* out, size_t groups) {
    CHECK(c, groups > 0 && groups <= 4096, "groups %zu (1..4096)", groups);
    CHECK(c, a && b && acc && out, "null operand");
    const size_t na = groups * 64, nc = groups * 32 * 64;
    int rc = ensure_tmp(c, 2 * na + 2 * nc);
    if (rc) return rc;
    float* da = (float*)c->tmp;
    float* db = da + na;
    float* dc = db + na;
    float* dout = dc + nc;
    HIPCHK(c, hipMemcpyAsync(da, a, na * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(db, b, na * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(dc, acc, nc * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, kr::launch_mfma_f32_probe(c->stream, da, db, dc, dout, groups));
    HIPCHK(c, hipMemcpyAsync(out, dout, nc * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_dbg_serial_sum(kr_ctx* c, const float* values, size_t n, size_t count, int waves, uint32_t* out) {
    CHECK(c, waves == 1 || waves == 2 || waves == 4 || waves == 16, "waves %d (1, 2, 4 or 16)", waves);
    CHECK(c, n >= 1 && n <= 2048, "n %zu (1..2048)", n);
    CHECK(c, count >= 1 && count <= 65536, "count %zu (1..65536)", count);
    CHECK(c, values && out, "null operand");
    int rc = ensure_tmp(c, n * count + 5 * count);
    if (rc) return rc;
    float* dx = (float*)c->tmp;
    uint32_t* dout = (uint32_t*)(dx + n * count);
    HIPCHK(c, hipMemcpyAsync(dx, values, n * count * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, kr::launch_serial_sum_probe(c->stream, dx, n, count, waves, dout));
    HIPCHK(c, hipMemcpyAsync(out, dout, 5 * count * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_matrix_shape(kr_ctx* c, kr_mat w, size_t* out_dim, size_t* in_dim, int* storage) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    *out_dim = m->m.n;
    *in_dim = m->m.k;
    *storage = m->m.storage;
    return KR_OK;
}

int kr_matrix_read(kr_ctx* c, kr_mat w, int8_t* quants, size_t quants_bytes, void* scales, size_t scales_bytes) {
    Mat* m = mat_of(c, w);
    CHECK(c, m != nullptr, "unknown matrix %u", (unsigned)w);
    const size_t nk = m->m.n * m->m.k, ns = m->m.n * (m->m.k / 32) * (m->m.storage == KR_STORAGE_Q8_0 ? 4 : 2);
    CHECK(c, quants_bytes == nk && scales_bytes == ns,
          "matrix %u holds %zu quant and %zu scale bytes; the buffers hold %zu and %zu", (unsigned)w, nk, ns,
          quants_bytes, scales_bytes);
    HIPCHK(c, hipMemcpyAsync(quants, m->m.q, nk, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(scales, m->m.s, ns, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

int kr_kv_synthetic(kr_ctx* c, size_t slots, uint64_t seed) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    CHECK(c, slots <= c->seq_len, "slots beyond seq_len");
    size_t per = slots * c->kv_dim;
    for (size_t l = 0; l < c->n_layers; l++) {
        size_t off = l * c->seq_len * c->kv_dim;
        HIPCHK(c, kr::launch_synthetic_normal(c->stream, c->kc + off, per, seed * 1000003ull + 2 * l));
        HIPCHK(c, kr::launch_synthetic_normal(c->stream, c->vc + off, per, seed * 1000003ull + 2 * l + 1));
    }
    return KR_OK;
}

int kr_argmax(kr_ctx* c, kr_buf x, size_t len, size_t index) {
    BUF(xb, x, len);
    CHECK(c, len > 0, "argmax of an empty buffer");
    CHECK(c, index < kr_ctx::kTokens, "token index %zu out of range", index);
    HIPCHK(c, kr::launch_argmax(c->stream, xb->p, len, c->tokens + index));
    return KR_OK;
}

int kr_read_tokens(kr_ctx* c, size_t* out, size_t n) {
    CHECK(c, n <= kr_ctx::kTokens, "too many tokens");
    std::vector<uint32_t> t(n);
    if (n) HIPCHK(c, hipMemcpyAsync(t.data(), c->tokens, n * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    for (size_t i = 0; i < n; i++) out[i] = t[i];
    return KR_OK;
}

int kr_synchronize(kr_ctx* c) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KR_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Device-step entry points for the model driver (internal.hpp).
namespace kri {

hipStream_t stream(kr_ctx* c) { return c->stream; }

int set_error(kr_ctx* c, int code, const char* msg) { return fail(c, code, "%s", msg); }

int device_u32(kr_ctx* c, size_t n, uint32_t** out) {
    *out = nullptr;
    HIPCHK(c, hipMalloc(out, n * sizeof(uint32_t)));
    HIPCHK(c, hipMemsetAsync(*out, 0, n * sizeof(uint32_t), c->stream));
    return KR_OK;
}

void device_free(void* p) {
    if (p) (void)hipFree(p);
}

uint32_t* token_ring(kr_ctx* c) { return c->tokens; }
uint64_t epoch(kr_ctx* c) { return c->epoch; }
size_t token_ring_len() { return kr_ctx::kTokens; }

int embed_rows(kr_ctx* c, const size_t* tokens, size_t n, kr_buf out) {
    Mat* e = mat_of(c, c->embedding);
    CHECK(c, c->prepared && e != nullptr, "prepare() runs before any compute");
    BUF(o, out, n * e->m.k);
    std::vector<uint32_t> t(n);
    for (size_t i = 0; i < n; i++) {
        CHECK(c, tokens[i] < e->m.n, "token %zu out of range (vocab %zu)", tokens[i], e->m.n);
        t[i] = (uint32_t)tokens[i];
    }
    const uint32_t* td;
    int rc = stage(c, c->st_tok, t.data(), n, &td);
    if (rc) return rc;
    HIPCHK(c, kr::launch_embed_rows(c->stream, e->m, td, n, o->p));
    return KR_OK;
}

int embed_dev(kr_ctx* c, const uint32_t* token_dev, kr_buf out, size_t offset) {
    Mat* e = mat_of(c, c->embedding);
    CHECK(c, c->prepared && e != nullptr, "prepare() runs before any compute");
    BUF(o, out, offset + e->m.k);
    HIPCHK(c, kr::launch_embed(c->stream, e->m, 0, token_dev, o->p + offset));
    return KR_OK;
}

int rope_dev(kr_ctx* c, kr_buf q, kr_buf k, size_t qw, size_t kvw, const uint32_t* pos_dev, const kr_rope_spec* spec) {
    CHECK(c, spec && spec->head_size >= 2 && spec->head_size % 2 == 0, "rope head_size must be even");
    BUF(qb, q, qw);
    BUF(kb, k, kvw);
    const float2* tab;
    int rc = rope_table(c, spec->theta, spec->head_size, c->seq_len, &tab);  // covers every slot
    if (rc) return rc;
    HIPCHK(c, kr::launch_rope(c->stream, qb->p, kb->p, qw, kvw, 1, pos_dev, tab, spec->head_size, spec->interleaved));
    return KR_OK;
}

int kv_write_dev(kr_ctx* c, size_t layer, const uint32_t* slot_dev, kr_buf k, kr_buf v) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    BUF(kb, k, c->kv_dim);
    BUF(vb, v, c->kv_dim);
    HIPCHK(c, kr::launch_kv_write(c->stream, c->kc, c->vc, layer, c->seq_len, c->kv_dim, slot_dev, kb->p, vb->p, 1));
    return KR_OK;
}

int attention_dev(kr_ctx* c, kr_buf q, kr_buf out, kr_buf att, size_t layer, const uint32_t* window_dev,
                  const kr_attn_spec* sp) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    CHECK(c, sp && sp->kv_dim == c->kv_dim && sp->seq_len == c->seq_len,
          "attention spec does not match the prepared cache");
    size_t width = sp->n_heads * sp->head_size;
    BUF(qb, q, width);
    BUF(ob, out, width);
    BUF(ab, att, sp->n_heads * sp->seq_len);
    float scale = 1.0f / sqrtf((float)sp->head_size);
    HIPCHK(c, kr::launch_attention(c->stream, qb->p, ob->p, ab->p, c->kc, c->vc, layer,
                                   (const kr::DevWindow*)window_dev, 1, c->seq_len, sp->n_heads, sp->kv_mul,
                                   sp->head_size, sp->kv_dim, sp->seq_len, scale));
    return KR_OK;
}

int norm_quant(kr_ctx* c, kr_buf x, kr_buf add, int add_planes, kr_buf w, kr_buf out, size_t rows, size_t dim,
               float eps, bool chain_major) {
    CHECK(c, dim % 32 == 0 && dim <= 8000, "fused norm needs dim %% 32 == 0 and dim <= 8000 (got %zu)", dim);
    CHECK(c, add_planes == 1 || add_planes == 4, "an added projection comes as 1 or 4 planes");
    CHECK(c, !chain_major || dim % 128 == 0, "chain-major blocks need dim %% 128 == 0");
    BUF(xb, x, rows * dim);
    BUF(wb, w, dim);
    BUF(ob, out, rows * dim);
    const float* ap = nullptr;
    if (add != KR_NO_BUF) {
        BUF(ab, add, add_planes * rows * dim);
        ap = ab->p;
    }
    int rc = ensure_workspace(c, rows, dim);
    if (rc) return rc;
    HIPCHK(c, kr::launch_add_rms_quant(c->stream, xb->p, ap, wb->p, ob->p, rows, dim, eps, c->wq, c->ws, c->wh,
                                       add_planes, chain_major));
    c->q_rows = rows;
    c->q_width = dim;
    c->q_chain_major = chain_major;
    return KR_OK;
}

int add_planes(kr_ctx* c, kr_buf dst, kr_buf planes, size_t len) {
    BUF(d, dst, len);
    BUF(p, planes, 4 * len);
    HIPCHK(c, kr::launch_add_planes(c->stream, d->p, p->p, len));
    return KR_OK;
}


int project_q(kr_ctx* c, size_t layer, const int* projs, const kr_buf* ys, int n, size_t rows) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    CHECK(c, n >= 1 && n <= 3, "1 to 3 projections per launch");
    const DevMatrix* ms[3];
    float* yp[3];
    bool same = true;
    for (int i = 0; i < n; i++) {
        const Mat* m = proj_mat(c, layer, projs[i]);
        CHECK(c, m != nullptr, "projection %d is not live on layer %zu", projs[i], layer);
        ms[i] = &m->m;
        CHECK(c, rows <= c->q_rows && ms[i]->k == c->q_width && !c->q_chain_major,
              "the workspace holds %zu rows of %zu, not %zu of %zu", c->q_rows, c->q_width, rows, ms[i]->k);
        BUF(yb, ys[i], rows * ms[i]->n);
        yp[i] = yb->p;
        same = same && ms[i]->storage == ms[0]->storage;
    }
    if (rows == 0) return KR_OK;
    if (same) {
        HIPCHK(c, kr::launch_project_set(c->stream, sem_for_project(*ms[0]), ms, yp, n, act(c), rows, nullptr));
    } else {
        for (int i = 0; i < n; i++)
            HIPCHK(c, kr::launch_project(c->stream, sem_for_project(*ms[i]), *ms[i], act(c), rows, yp[i], ms[i]->n,
                                         nullptr));
    }
    return KR_OK;
}

// The FFN of a prefill batch after the norm's quantization (the workspace
// holds `rows` rows of in_dim): gate and up as one Q8_0 GEMM whose epilogue
// forms h = SiLU(gate) * up and h's Q8 blocks (silu_quant's arithmetic) into
// the second workspace, then down from there into `out` -- the bits of
// project_q(gate, up), silu_quant and project_q(down), one launch fewer and
// no f32 gate/up round trip. The workspace still holds the norm's rows after.
bool ffn_swiglu_ok(kr_ctx* c, size_t layer, size_t rows) {
    if (!c->prepared || layer >= c->n_layers || rows < 8) return false;
    const Mat* g = proj_mat(c, layer, KR_PROJ_GATE);
    const Mat* u = proj_mat(c, layer, KR_PROJ_UP);
    const Mat* d = proj_mat(c, layer, KR_PROJ_DOWN);
    return g && u && d && g->m.storage == KR_STORAGE_Q8_0 && u->m.storage == KR_STORAGE_Q8_0 &&
           g->m.n == u->m.n && g->m.k == u->m.k && g->m.n % 32 == 0 && d->m.k == g->m.n &&
           sem_for_project(g->m) == kr::SEM_FOUR_PARTIALS_F32 && rows <= c->q_rows && g->m.k == c->q_width &&
           !c->q_chain_major;
}

int ffn_swiglu_down(kr_ctx* c, size_t layer, size_t rows, kr_buf out, int max_planes, int* planes) {
    CHECK(c, ffn_swiglu_ok(c, layer, rows), "the fused gate/up + SiLU GEMM does not apply to layer %zu", layer);
    const Mat* g = proj_mat(c, layer, KR_PROJ_GATE);
    const Mat* u = proj_mat(c, layer, KR_PROJ_UP);
    const Mat* d = proj_mat(c, layer, KR_PROJ_DOWN);
    const bool split = max_planes == 4 && chain_split_ok(d->m, rows);
    BUF(ob, out, (split ? 4 : 1) * rows * d->m.n);
    int rc = ensure_workspace2(c, rows, g->m.n);
    if (rc) return rc;
    const DevMatrix* dc = nullptr;
    if (split && (rc = ensure_chain_major(c, d, &dc)) != KR_OK) return rc;
    HIPCHK(c, kr::launch_gate_up_silu_q8(c->stream, g->m, u->m, act(c), rows, c->wq2, c->ws2, c->wh2, split));
    const kr::QuantAct h{c->wq2, c->ws2, c->wh2};
    if (split)
        HIPCHK(c, kr::launch_gemm_q8_cs(c->stream, *dc, h, rows, ob->p));
    else
        HIPCHK(c, kr::launch_project(c->stream, sem_for_project(d->m), d->m, h, rows, ob->p, d->m.n, nullptr));
    *planes = split ? 4 : 1;
    return KR_OK;
}

int silu_quant(kr_ctx* c, kr_buf gate, kr_buf up, size_t rows, size_t width) {
    CHECK(c, width % 32 == 0, "fused silu needs width %% 32 == 0");
    BUF(g, gate, rows * width);
    BUF(u, up, rows * width);
    int rc = ensure_workspace(c, rows, width);
    if (rc) return rc;
    HIPCHK(c, kr::launch_silu_quant(c->stream, g->p, u->p, rows, width, c->wq, c->ws, c->wh));
    c->q_rows = rows;
    c->q_width = width;
    c->q_chain_major = false;
    return KR_OK;
}

int rope_kv(kr_ctx* c, kr_buf q, kr_buf k, kr_buf v, size_t qw, size_t kvw, size_t rows, const size_t* pos_host,
            const size_t* slot_host, const uint32_t* pos_dev, size_t layer, const kr_rope_spec* spec, kr_buf nq,
            kr_buf nk, float eps) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    const bool norms = nq != KR_NO_BUF || nk != KR_NO_BUF;
    CHECK(c, !norms || (nq != KR_NO_BUF && nk != KR_NO_BUF), "the fused q/k norms take both weights");
    CHECK(c, spec && spec->head_size >= 2 && spec->head_size % 2 == 0, "rope head_size must be even");
    CHECK(c, kvw == c->kv_dim && kvw % spec->head_size == 0 && qw % spec->head_size == 0,
          "fused rope/kv_write needs whole heads and kv_width == kv_dim");
    BUF(qb, q, rows * qw);
    BUF(kb, k, rows * kvw);
    BUF(vb, v, rows * kvw);
    if (rows == 0) return KR_OK;
    const uint32_t* pd;
    const uint32_t* sd;
    const float2* tab;
    int rc;
    if (pos_dev) {
        CHECK(c, rows == 1, "device positions are for one row");
        rc = rope_table(c, spec->theta, spec->head_size, c->seq_len, &tab);
        if (rc) return rc;
        pd = pos_dev;
        sd = pos_dev;
    } else {
        size_t maxp = 0;
        for (size_t i = 0; i < rows; i++) {
            maxp = pos_host[i] > maxp ? pos_host[i] : maxp;
            CHECK(c, slot_host[i] < c->seq_len, "slot %zu out of range", slot_host[i]);
        }
        CHECK(c, maxp < (1u << 24), "rope position %zu too large", maxp);
        rc = rope_table(c, spec->theta, spec->head_size, maxp + 1, &tab);
        if (rc) return rc;
        std::vector<uint32_t> p = to_u32(pos_host, rows), sl = to_u32(slot_host, rows);
        rc = stage(c, c->st_pos, p.data(), rows, &pd);
        if (rc) return rc;
        rc = stage(c, c->st_slots, sl.data(), rows, &sd);
        if (rc) return rc;
    }
    if (norms) {
        CHECK(c, spec->head_size <= 128 && spec->head_size % 4 == 0,
              "the fused q/k norms take head sizes that are multiples of 4, at most 128");
        BUF(wqb, nq, spec->head_size);
        BUF(wkb, nk, spec->head_size);
        HIPCHK(c, kr::launch_qk_norm_rope_kv(c->stream, qb->p, kb->p, vb->p, qw, kvw, rows, wqb->p, wkb->p, eps, pd,
                                             sd, tab, spec->head_size, spec->interleaved, c->kc, c->vc, layer,
                                             c->seq_len));
        return KR_OK;
    }
    HIPCHK(c, kr::launch_rope_kv(c->stream, qb->p, kb->p, vb->p, qw, kvw, rows, pd, sd, tab, spec->head_size,
                                 spec->interleaved, c->kc, c->vc, layer, c->seq_len));
    return KR_OK;
}

bool qkv_rope_ok(kr_ctx* c, size_t layer, size_t rows, const kr_rope_spec* spec) {
    if (!c->prepared || layer >= c->n_layers || !spec || spec->head_size != 64 || spec->interleaved) return false;
    const Mat* q = proj_mat(c, layer, KR_PROJ_Q);
    const Mat* k = proj_mat(c, layer, KR_PROJ_K);
    const Mat* v = proj_mat(c, layer, KR_PROJ_V);
    return q && k && v && k->m.n == c->kv_dim && rows <= c->q_rows && q->m.k == c->q_width && !c->q_chain_major &&
           kr::qkv_rope_q8_ok(q->m, k->m, v->m, rows);
}

int project_qkv_rope(kr_ctx* c, size_t layer, kr_buf q, size_t rows, const size_t* pos_host, const size_t* slot_host,
                     const kr_rope_spec* spec) {
    CHECK(c, qkv_rope_ok(c, layer, rows, spec), "the q/k/v GEMM with RoPE does not apply to layer %zu", layer);
    const Mat* qm = proj_mat(c, layer, KR_PROJ_Q);
    const Mat* km = proj_mat(c, layer, KR_PROJ_K);
    const Mat* vm = proj_mat(c, layer, KR_PROJ_V);
    BUF(qb, q, rows * qm->m.n);
    size_t maxp = 0;
    for (size_t i = 0; i < rows; i++) {
        maxp = pos_host[i] > maxp ? pos_host[i] : maxp;
        CHECK(c, slot_host[i] < c->seq_len, "slot %zu out of range", slot_host[i]);
    }
    CHECK(c, maxp < (1u << 24), "rope position %zu too large", maxp);
    const float2* tab;
    int rc = rope_table(c, spec->theta, spec->head_size, maxp + 1, &tab);
    if (rc) return rc;
    const uint32_t* pd;
    const uint32_t* sd;
    std::vector<uint32_t> p = to_u32(pos_host, rows), sl = to_u32(slot_host, rows);
    if ((rc = stage(c, c->st_pos, p.data(), rows, &pd)) != KR_OK) return rc;
    if ((rc = stage(c, c->st_slots, sl.data(), rows, &sd)) != KR_OK) return rc;
    const size_t base = layer * c->seq_len * c->kv_dim;
    HIPCHK(c, kr::launch_qkv_rope_q8(c->stream, qm->m, km->m, vm->m, act(c), rows, qb->p, pd, sd, tab, c->kc + base,
                                     c->vc + base));
    return KR_OK;
}

int attention_quant(kr_ctx* c, kr_buf q, kr_buf out, kr_buf att, size_t layer, const kr_window* windows, size_t n,
                    const uint32_t* window_dev, const kr_attn_spec* sp, bool keep_att) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    CHECK(c, sp && sp->kv_dim == c->kv_dim && sp->seq_len == c->seq_len,
          "attention spec does not match the prepared cache");
    CHECK(c, sp->head_size % 32 == 0 && sp->head_size <= 256, "fused attention needs head_size %% 32 == 0");
    CHECK(c, sp->kv_mul > 0 && sp->n_heads % sp->kv_mul == 0 && (sp->n_heads / sp->kv_mul) * sp->head_size <= sp->kv_dim,
          "attention geometry is inconsistent");
    size_t width = sp->n_heads * sp->head_size;
    BUF(qb, q, n * width);
    BUF(ob, out, n * width);
    BUF(ab, att, n * sp->n_heads * sp->seq_len);
    if (n == 0) return KR_OK;
    const uint32_t* wd;
    size_t max_count;
    std::vector<uint32_t> w;  // host copy of the windows, read by launch_attention
    if (window_dev) {
        CHECK(c, n == 1, "a device window is for one row");
        wd = window_dev;
        max_count = c->seq_len;
    } else {
        w.resize(4 * n);
        max_count = 0;
        for (size_t i = 0; i < n; i++) {
            const kr_window& x = windows[i];
            CHECK(c, x.att_start <= x.slot && x.slot < c->seq_len && x.shared_start <= x.shared_end &&
                         x.shared_end <= c->seq_len,
                  "window %zu out of range", i);
            size_t count = (x.shared_end - x.shared_start) + x.slot - x.att_start + 1;
            CHECK(c, count <= c->seq_len, "window %zu attends more than seq_len slots", i);
            max_count = count > max_count ? count : max_count;
            w[4 * i] = (uint32_t)x.att_start;
            w[4 * i + 1] = (uint32_t)x.slot;
            w[4 * i + 2] = (uint32_t)x.shared_start;
            w[4 * i + 3] = (uint32_t)x.shared_end;
        }
        int rc = stage(c, c->st_win, w.data(), 4 * n, &wd);
        if (rc) return rc;
    }
    int rc = ensure_workspace(c, n, width);
    if (rc) return rc;
    if (w.empty()) {  // one device window
        float scale = 1.0f / sqrtf((float)sp->head_size);
        HIPCHK(c, kr::launch_attention(c->stream, qb->p, ob->p, ab->p, c->kc, c->vc, layer, (const kr::DevWindow*)wd,
                                       n, max_count, sp->n_heads, sp->kv_mul, sp->head_size, sp->kv_dim, sp->seq_len,
                                       scale, c->wq, c->ws, c->wh));
    } else {
        rc = attention_many(c, qb->p, ob->p, ab->p, layer, wd, w, n, max_count, sp, c->wq, c->ws, c->wh, keep_att);
        if (rc) return rc;
    }
    c->q_rows = n;
    c->q_width = width;
    c->q_chain_major = false;
    return KR_OK;
}

int logits_q(kr_ctx* c, kr_buf y) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    Mat* mt = mat_of(c, c->classifier != KR_NO_MAT ? c->classifier : c->embedding);
    CHECK(c, mt != nullptr, "no classifier bound");
    const DevMatrix* m;
    int sem;
    int rc = classifier_matrix(c, mt, &m, &sem);
    if (rc) return rc;
    CHECK(c, c->q_rows >= 1 && c->q_width == m->k && !c->q_chain_major,
          "the workspace does not hold the classifier input");
    BUF(yb, y, m->n);
    HIPCHK(c, kr::launch_project(c->stream, sem, *m, act(c), 1, yb->p, m->n, nullptr));
    return KR_OK;
}

// The fused decode producers (launch_project_pro): one row, M = 1.
bool pro_fusable(size_t k) { return k % 32 == 0 && k <= 8192 && 8192 / k * (k / 16) <= 512; }

int norm_project(kr_ctx* c, size_t layer, const int* projs, const kr_buf* ys, int n, kr_buf x, kr_buf add, kr_buf w,
                 kr_buf x_out, size_t dim, float eps) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    CHECK(c, n >= 1 && n <= 3 && pro_fusable(dim), "fused norm + projection: 1-3 matrices, dim %zu", dim);
    const DevMatrix* ms[3];
    float* yp[3];
    for (int i = 0; i < n; i++) {
        const Mat* m = proj_mat(c, layer, projs[i]);
        CHECK(c, m != nullptr, "projection %d is not live on layer %zu", projs[i], layer);
        ms[i] = &m->m;
        CHECK(c, ms[i]->k == dim && ms[i]->storage == ms[0]->storage, "fused projections share in_dim and storage");
        BUF(yb, ys[i], ms[i]->n);
        yp[i] = yb->p;
    }
    BUF(xb, x, dim);
    BUF(wb, w, dim);
    BUF(ob, x_out, dim);
    CHECK(c, x_out != x, "the updated residual goes to a second buffer");
    const float* ap = nullptr;
    if (add != KR_NO_BUF) {
        BUF(ab, add, dim);
        ap = ab->p;
    }
    HIPCHK(c, kr::launch_project_pro(c->stream, sem_for_project(*ms[0]), ms, yp, n, 1, xb->p, ap, wb->p, ob->p, eps));
    return KR_OK;
}

// the per-head RMSNorms of q and k (qk-norm models) in one launch
int qk_norm_pair(kr_ctx* c, kr_buf q, kr_buf k, size_t rows, size_t q_width, size_t k_width, size_t head,
                 kr_buf wq, kr_buf wk, float eps) {
    CHECK(c, head > 0 && head <= 256, "head_size must be in 1..=256");
    BUF(qb, q, rows * q_width);
    BUF(kb, k, rows * k_width);
    BUF(wqb, wq, head);
    BUF(wkb, wk, head);
    HIPCHK(c, kr::launch_qk_norm(c->stream, qb->p, rows, q_width, head, wqb->p, eps, kb->p, k_width, wkb->p));
    return KR_OK;
}

// y = C * conv(B * x) of one LFM2 decode row (k_conv_block_decode)
int conv_block_decode(kr_ctx* c, kr_buf y, kr_buf bcx, kr_buf kernel, kr_buf state, size_t dim, size_t k) {
    CHECK(c, k >= 1, "conv kernel width must be positive");
    BUF(yb, y, dim);
    BUF(xb, bcx, 3 * dim);
    BUF(kb, kernel, dim * k);
    BUF(sb, state, (k - 1) * dim);
    CHECK(c, y != bcx, "the conv block writes a second buffer");
    HIPCHK(c, kr::launch_conv_block_decode(c->stream, yb->p, xb->p, kb->p, sb->p, dim, k));
    return KR_OK;
}

// The conv of `rows` rows of x as if they were fed one at a time through
// conv_decode (the ring supplies the history, then advances by `rows`).
int mul_rows(kr_ctx* c, kr_buf out, size_t oo, size_t os, kr_buf a, size_t ao, size_t as, kr_buf b, size_t bo,
             size_t bs, size_t rows, size_t n) {
    CHECK(c, out != a && out != b, "mul_rows: the output may not alias an input");
    if (rows == 0 || n == 0) return KR_OK;
    BUF(o, out, oo + (rows - 1) * os + n);
    BUF(ab, a, ao + (rows - 1) * as + n);
    BUF(bb, b, bo + (rows - 1) * bs + n);
    HIPCHK(c, kr::launch_mul_rows(c->stream, o->p + oo, os, ab->p + ao, as, bb->p + bo, bs, rows, n));
    return KR_OK;
}

int conv_prefill_stepped(kr_ctx* c, kr_buf out, kr_buf x, kr_buf kernel, kr_buf state, size_t rows, size_t dim,
                         size_t k) {
    CHECK(c, k >= 1 && k <= 16, "conv kernel width %zu outside 1..16", k);
    BUF(o, out, rows * dim);
    BUF(xb, x, rows * dim);
    BUF(kb, kernel, dim * k);
    BUF(sb, state, (k - 1) * dim);
    CHECK(c, out != x && out != state && x != state, "conv_prefill_stepped buffers must be distinct");
    HIPCHK(c, kr::launch_conv_prefill(c->stream, o->p, xb->p, kb->p, rows, dim, k, sb->p));
    HIPCHK(c, kr::launch_conv_ring_advance(c->stream, sb->p, xb->p, rows, dim, k));
    return KR_OK;
}

// Decode gate/up of one row with the norm in front and SiLU(gate) * up + Q8
// behind (k_gemv_swiglu): the down projection's input lands in the
// activation workspace; h (f32) goes to `h`.
bool swiglu_ok(kr_ctx* c, size_t layer, size_t dim) {
    if (!c->prepared || layer >= c->n_layers) return false;
    const Mat* g = proj_mat(c, layer, KR_PROJ_GATE);
    const Mat* u = proj_mat(c, layer, KR_PROJ_UP);
    return g && u && g->m.k == dim && kr::swiglu_fusable(g->m, u->m);
}

int norm_swiglu(kr_ctx* c, size_t layer, kr_buf x, kr_buf add, kr_buf w, kr_buf x_out, kr_buf h, size_t dim,
                float eps) {
    CHECK(c, swiglu_ok(c, layer, dim), "fused gate/up + SwiGLU does not apply to layer %zu", layer);
    const Mat* g = proj_mat(c, layer, KR_PROJ_GATE);
    const Mat* u = proj_mat(c, layer, KR_PROJ_UP);
    const size_t hidden = g->m.n;
    BUF(xb, x, dim);
    BUF(wb, w, dim);
    BUF(ob, x_out, dim);
    BUF(hb, h, hidden);
    CHECK(c, x_out != x, "the updated residual goes to a second buffer");
    const float* ap = nullptr;
    if (add != KR_NO_BUF) {
        BUF(ab, add, dim);
        ap = ab->p;
    }
    int rc = ensure_workspace(c, 1, hidden);
    if (rc) return rc;
    HIPCHK(c, kr::launch_gate_up_swiglu(c->stream, sem_for_project(g->m), g->m, u->m, xb->p, ap, wb->p, ob->p, eps,
                                        c->wq, c->ws, c->wh, hb->p));
    c->q_rows = 1;
    c->q_width = hidden;
    c->q_chain_major = false;
    return KR_OK;
}

bool split_attention_ok(kr_ctx* c, const kr_attn_spec* sp, size_t max_count) {
    return sp && c->prepared && sp->seq_len == c->seq_len && max_count >= 1 && max_count <= c->seq_len &&
           kr::attention_split_ok(max_count, sp->kv_mul, sp->head_size);
}

int rope_attention(kr_ctx* c, kr_buf q, kr_buf k, kr_buf v, kr_buf out, kr_buf att, size_t layer, size_t pos_host,
                   const uint32_t* step_dev, const kr_attn_spec* sp, const kr_rope_spec* rs, size_t dev_max_count,
                   kr_buf nq, kr_buf nk, float eps) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    const size_t cap = step_dev ? dev_max_count : pos_host + 1;
    CHECK(c, split_attention_ok(c, sp, cap) && sp->kv_dim == c->kv_dim && sp->n_heads % sp->kv_mul == 0,
          "split decode attention does not apply to this geometry");
    CHECK(c, rs && rs->head_size == sp->head_size, "rope and attention head sizes differ");
    const size_t width = sp->n_heads * sp->head_size;
    BUF(qb, q, width);
    BUF(kb, k, c->kv_dim);
    BUF(vb, v, c->kv_dim);
    BUF(ob, out, width);
    BUF(ab, att, sp->n_heads * sp->seq_len);
    const float* wq = nullptr;
    const float* wk = nullptr;
    if (nq != KR_NO_BUF) {
        BUF(wqb, nq, sp->head_size);
        wq = wqb->p;
    }
    if (nk != KR_NO_BUF) {
        BUF(wkb, nk, sp->head_size);
        wk = wkb->p;
    }
    int rc0 = ensure_attn_scratch(c, kr::attention_split_scratch(sp->n_heads, c->seq_len));
    if (rc0) return rc0;
    const float2* tab;
    const uint32_t* wd;
    const uint32_t* pd;
    size_t max_count;
    int rc;
    if (step_dev) {  // window at step[1..4], position (== slot) at step[2]
        rc = rope_table(c, rs->theta, rs->head_size, cap, &tab);
        if (rc) return rc;
        wd = step_dev + 1;
        pd = step_dev + 2;
        max_count = cap;
    } else {
        CHECK(c, pos_host < c->seq_len, "position %zu out of range", pos_host);
        rc = rope_table(c, rs->theta, rs->head_size, pos_host + 1, &tab);
        if (rc) return rc;
        uint32_t w[4] = {0, (uint32_t)pos_host, 0, 0};
        rc = stage(c, c->st_win, w, 4, &wd);
        if (rc) return rc;
        uint32_t p = (uint32_t)pos_host;
        rc = stage(c, c->st_pos, &p, 1, &pd);
        if (rc) return rc;
        max_count = pos_host + 1;
    }
    const float scale = 1.0f / sqrtf((float)sp->head_size);  // cpu.rs:591
    HIPCHK(c, kr::launch_attention_split(c->stream, qb->p, kb->p, vb->p, ob->p, ab->p, c->kc, c->vc, layer,
                                         (const kr::DevWindow*)wd, pd, tab, rs->interleaved, max_count, sp->n_heads,
                                         sp->kv_mul, sp->head_size, c->kv_dim, c->seq_len, scale, c->attn_scratch,
                                         wq, wk, eps));
    return KR_OK;
}

int quant_project(kr_ctx* c, size_t layer, int proj, kr_buf x, kr_buf y, size_t width) {
    CHECK(c, c->prepared && layer < c->n_layers, "layer %zu out of range", layer);
    CHECK(c, pro_fusable(width), "fused quantize + projection: width %zu", width);
    const Mat* m = proj_mat(c, layer, proj);
    CHECK(c, m != nullptr && m->m.k == width, "projection %d is not live on layer %zu", proj, layer);
    BUF(xb, x, width);
    BUF(yb, y, m->m.n);
    const DevMatrix* ms = &m->m;
    float* yp = yb->p;
    HIPCHK(c, kr::launch_project_pro(c->stream, sem_for_project(m->m), &ms, &yp, 1, 3, xb->p, nullptr, nullptr,
                                     nullptr, 0.0f));
    return KR_OK;
}

int logits_rows(kr_ctx* c, kr_buf y, size_t rows) {
    CHECK(c, c->prepared, "prepare() runs before any compute");
    Mat* mt = mat_of(c, c->classifier != KR_NO_MAT ? c->classifier : c->embedding);
    CHECK(c, mt != nullptr, "no classifier bound");
    const DevMatrix* m;
    int sem;
    int rc = classifier_matrix(c, mt, &m, &sem);
    if (rc) return rc;
    CHECK(c, c->q_rows >= rows && c->q_width == m->k && !c->q_chain_major,
          "the workspace does not hold the classifier input");
    BUF(yb, y, rows * m->n);
    HIPCHK(c, kr::launch_project(c->stream, sem, *m, act(c), rows, yb->p, m->n, nullptr));
    return KR_OK;
}

int greedy_step(kr_ctx* c, kr_buf logits, size_t len, uint32_t* step) {
    BUF(l, logits, len);
    CHECK(c, len > 0, "argmax of an empty buffer");
    Mat* e = mat_of(c, c->embedding);
    CHECK(c, e != nullptr && len <= e->m.n, "greedy tokens must index the embedding (vocab %zu)", len);
    HIPCHK(c, kr::launch_greedy_step(c->stream, l->p, len, step, c->tokens, kr_ctx::kTokens));
    return KR_OK;
}

}  // namespace kri
