// hq_api.hip - C ABI of the gfx950 quantized matmul path (include/hq.h): weight residency,
// argument checking and kernel dispatch. Every entry point validates shapes, alignment and ids on
// the host before a kernel is launched, so no launch can read or write outside its buffers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <thread>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

#include "hq.h"
#include "hq_llama.h"
#include "hq_internal.h"
#include "hq_kernels.h"

struct hq_mat {
    hq_dev_mat m;
    int device;
    void *alloc;
    size_t bytes;
    int pair;  // a gate/up pair matrix (hq_mat_upload_pair): rows 16k .. 16k + 7 gate, + 8 .. + 15 up
};

// ------------------------------------------------------------------------------------ errors
static thread_local char g_err[512] = "";

static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

#define HIPCK(call)                                                                                         \
    do {                                                                                                    \
        hipError_t e_ = (call);                                                                             \
        if (e_ != hipSuccess) return fail("HIP %s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, \
                                          __LINE__);                                                        \
    } while (0)

extern "C" const char *hq_last_error(void) { return g_err; }

extern "C" int hq_internal_fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

// ------------------------------------------------------------------------------------ device
static int use_device(int device) {
    int cur = -1;
    HIPCK(hipGetDevice(&cur));
    if (cur != device) HIPCK(hipSetDevice(device));
    return 0;
}

extern "C" int hq_device_count(int *count) {
    HIPCK(hipGetDeviceCount(count));
    return 0;
}

extern "C" int hq_device_name(int device, char *name, size_t name_len, char *arch, size_t arch_len) {
    hipDeviceProp_t p;
    HIPCK(hipGetDeviceProperties(&p, device));
    if (name && name_len) snprintf(name, name_len, "%s", p.name);
    if (arch && arch_len) snprintf(arch, arch_len, "%s", p.gcnArchName);
    return 0;
}

extern "C" int hq_device_init(int device) {
    int n = 0;
    HIPCK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail("hq: device %d not found (%d visible)", device, n);
    HIPCK(hipSetDevice(device));
    hipDeviceProp_t p;
    HIPCK(hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail("hq: device %d is %s; this library is built for gfx950 (MI355X)", device, p.gcnArchName);
    return 0;
}

// ------------------------------------------------------------------------------------ residency
static uint32_t block_values(int t) {
    switch (t) {
    case HQ_GGML_Q8_0: return 32u;
    case HQ_GGML_Q2_K: case HQ_GGML_Q3_K: case HQ_GGML_Q4_K: case HQ_GGML_Q5_K: case HQ_GGML_Q6_K: return 256u;
    default: return 0u;
    }
}
static uint32_t block_bytes(int t) {
    switch (t) {
    case HQ_GGML_Q8_0: return 34u;
    case HQ_GGML_Q2_K: return 84u;
    case HQ_GGML_Q3_K: return 110u;
    case HQ_GGML_Q4_K: return 144u;
    case HQ_GGML_Q5_K: return 176u;
    case HQ_GGML_Q6_K: return 210u;
    default: return 0u;
    }
}
// Device bytes of one super-block where the GGUF block is padded into an aligned slot (the GGUF
// bytes, then zeros; every 16-byte load of a row aligned); 0 where the bytes are kept as they are.
static size_t slot_bytes(int t) { return t == HQ_GGML_Q2_K ? 96 : t == HQ_GGML_Q3_K ? 112 : t == HQ_GGML_Q6_K ? 224 : 0; }
static const char SUPPORTED[] = "Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14";

extern "C" int hq_internal_block_shape(int ggml_type, uint32_t *values, uint32_t *bytes) {
    if (!block_values(ggml_type)) return -1;
    *values = block_values(ggml_type);
    *bytes = block_bytes(ggml_type);
    return 0;
}

extern "C" const char *hq_internal_supported_types(void) { return SUPPORTED; }

// Storage row of Hugging Face row r (llama.cpp q/k interleave; reference src/model.c:283-289).
static uint32_t storage_row(uint32_t rows, uint32_t perm_heads, uint32_t r) {
    if (!perm_heads) return r;
    const uint32_t hd = rows / perm_heads, half = hd / 2, within = r % hd;
    return (r - within) + 2 * (within % half) + within / half;
}

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ------------------------------------------------------------------------------------ upload
// Matrices reach HBM through a per-device uploader: two pinned host staging buffers and two device
// staging buffers of UP_CHUNK bytes on a stream of its own. Chunk i of whole rows is copied (rows
// in Hugging Face order) from the caller's blocks (e.g. a mapped GGUF file) into pinned buffer i % 2
// by a few host threads, sent with an asynchronous host-to-device copy, and turned into the device
// layout by a repack kernel (Q8_0: quant and scale planes; Q6_K: 224-byte slots; Q4_K: copied into
// place directly), while the host already fills the other buffer.
namespace {
constexpr size_t UP_CHUNK = (size_t)32 << 20;

struct Uploader {
    hipStream_t st = nullptr;
    void *pinned[2] = {nullptr, nullptr}, *raw[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    std::mutex mu;  // one upload at a time per device
};
std::mutex g_up_mu;
std::map<int, Uploader *> g_up;

int uploader(int device, Uploader **out) {
    std::lock_guard<std::mutex> lk(g_up_mu);
    auto it = g_up.find(device);
    if (it != g_up.end()) {
        *out = it->second;
        return 0;
    }
    Uploader *u = new Uploader();
    hipError_t e = hipStreamCreateWithFlags(&u->st, hipStreamNonBlocking);
    for (int b = 0; b < 2 && e == hipSuccess; b++) {
        e = hipHostMalloc(&u->pinned[b], UP_CHUNK, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(&u->raw[b], UP_CHUNK);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&u->ev[b], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        for (int b = 0; b < 2; b++) {
            if (u->pinned[b]) (void)hipHostFree(u->pinned[b]);
            if (u->raw[b]) (void)hipFree(u->raw[b]);
            if (u->ev[b]) (void)hipEventDestroy(u->ev[b]);
        }
        if (u->st) (void)hipStreamDestroy(u->st);
        delete u;
        return fail("hq_mat_upload: staging buffers: %s", hipGetErrorString(e));
    }
    g_up[device] = u;
    *out = u;
    return 0;
}

// rows [r0, r0 + n) of a matrix into dst (rb bytes per row), row r read from row_ptr(r); split over
// a few host threads
template <class F>
void gather_rows(F row_ptr, size_t rb, uint32_t r0, uint32_t n, uint8_t *dst) {
    const size_t bytes = (size_t)n * rb;
    const int nthr = bytes >= ((size_t)8 << 20) ? 8 : 1;
    auto work = [&](int t) {
        const uint32_t a = (uint32_t)((uint64_t)n * t / nthr), b = (uint32_t)((uint64_t)n * (t + 1) / nthr);
        for (uint32_t r = a; r < b;) {
            // runs of rows that are consecutive in the source go in one copy
            const uint8_t *p = row_ptr(r0 + r);
            uint32_t e = r + 1;
            while (e < b && row_ptr(r0 + e) == p + (size_t)(e - r) * rb) e++;
            memcpy(dst + (size_t)r * rb, p, (size_t)(e - r) * rb);
            r = e;
        }
    };
    if (nthr == 1) {
        work(0);
        return;
    }
    // a thread that cannot be created (std::system_error under thread limits) leaves its share to
    // this thread, so the upload still completes instead of terminating the process
    std::vector<std::thread> th;
    int t = 1;
    try {
        th.reserve(nthr - 1);
        for (; t < nthr; t++) th.emplace_back(work, t);
    } catch (const std::exception &) {
    }
    for (int u = t; u < nthr; u++) work(u);
    work(0);
    for (auto &x : th) x.join();
}

// GGUF Q8_0 rows (34-byte blocks) -> quant plane bytes q ^ 0x80 and fp16 scale plane
__global__ void k_repack_q8_0(const uint8_t *__restrict__ raw, uint32_t n, uint32_t nb, uint32_t ldd, uint8_t *qs,
                              uint16_t *d) {
    const size_t total = (size_t)n * nb;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / nb, b = i % nb;
        const uint8_t *blk = raw + i * 34;
        d[r * ldd + b] = (uint16_t)(blk[0] | (blk[1] << 8));
        uint8_t *q = qs + r * (size_t)nb * 32 + b * 32;
#pragma unroll
        for (int j = 0; j < 32; j++) q[j] = blk[2 + j] ^ 0x80u;
    }
}

// GGUF k-quant rows (super-blocks of `in` halves, 2-byte aligned) -> slots of `out` halves (the tail
// zeroed): Q2_K 42 -> 48, Q3_K 55 -> 56, Q6_K 105 -> 112
__global__ void k_repack_slots(const uint16_t *__restrict__ raw, size_t nblk, uint32_t in, uint32_t out, uint16_t *dst) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < nblk * out; i += (size_t)gridDim.x * blockDim.x) {
        const size_t b = i / out, h = i % out;
        dst[i] = h < in ? raw[b * in + h] : (uint16_t)0;
    }
}

unsigned up_grid(size_t n) { return (unsigned)((n + 255) / 256 < 16384 ? (n + 255) / 256 : 16384); }
}  // namespace

// Checks shared by the upload entry points: a GGUF block type hq_mat_upload supports, whole blocks
// per row, the size limits; *rb = GGUF bytes per row.
static int check_wmat(const hq_wmat_t *w, const char *who, size_t *rb) {
    if (!w || !w->data) return fail("%s: no matrix", who);
    if (w->dtype != HQ_DT_GGML) return fail("%s: dtype %d is not a GGUF block type", who, w->dtype);
    const uint32_t per = block_values(w->ggml_type);
    if (!per) return fail("%s: ggml type %d is not supported (%s)", who, w->ggml_type, SUPPORTED);
    if (w->rows == 0 || w->cols == 0 || w->cols % per)
        return fail("%s: shape [%u, %u] is not a whole number of %u-value blocks per row", who, w->rows, w->cols, per);
    if (w->rows > (1u << 30) || w->cols > (1u << 24)) return fail("%s: shape [%u, %u] too large", who, w->rows, w->cols);
    if (w->perm_heads && (w->rows % w->perm_heads || (w->rows / w->perm_heads) % 2))
        return fail("%s: %u rows do not split into %u heads of even size", who, w->rows, w->perm_heads);
    *rb = (size_t)(w->cols / per) * block_bytes(w->ggml_type);
    return 0;
}

// A rows x cols matrix of `type` whose GGUF row r (Hugging Face order) is row_ptr(r), into the
// device layout through the uploader.
template <class F>
static int upload_rows(int type, uint32_t rows, uint32_t cols, F row_ptr, int device, const char *who, hq_mat **out) {
    *out = nullptr;
    const uint32_t per = block_values(type);
    const size_t rb = (size_t)(cols / per) * block_bytes(type);
    // the kernels address a matrix through 32-bit buffer ranges: its device bytes stay below 4 GiB
    const size_t K = cols, nb = K / per, ldd = round_up(K / 32, 8), qbytes = round_up((size_t)rows * K, 256);
    const size_t drb = slot_bytes(type) ? nb * slot_bytes(type) : rb;
    const size_t dev_bytes = type == HQ_GGML_Q8_0 ? qbytes + (size_t)rows * ldd * 2 : drb * rows;
    if (dev_bytes >= ((size_t)1 << 32))
        return fail("%s: shape [%u, %u] needs %zu device bytes; one matrix is limited to 4 GiB (split its rows)", who, rows,
                    cols, dev_bytes);
    // Q4_K: the GEMM kernels' per-super-block column tables follow the blocks (a third of their bytes)
    const size_t tab_at = round_up(dev_bytes, 256), tab_bytes = type == HQ_GGML_Q4_K ? (size_t)rows * nb * HQ_Q4K_TAB_BYTES : 0;
    if (rb > UP_CHUNK) return fail("%s: a row of %zu bytes exceeds the %zu-byte staging buffer", who, rb, UP_CHUNK);
    if (use_device(device)) return -1;
    Uploader *u;
    if (uploader(device, &u)) return -1;
    hq_mat *m = (hq_mat *)calloc(1, sizeof *m);
    if (!m) return fail("%s: out of host memory", who);
    m->device = device;
    m->m.type = type;
    m->m.rows = rows;
    m->m.cols = cols;
    m->m.row_bytes = drb;
    m->m.ldd = type == HQ_GGML_Q8_0 ? (int)ldd : 0;
    m->bytes = tab_bytes ? tab_at + tab_bytes + HQ_Q4K_TAB_PAD : dev_bytes;
    hipError_t e = hipMalloc(&m->alloc, m->bytes);
    if (e != hipSuccess) {
        free(m);
        return fail("%s: hipMalloc(%zu) failed: %s", who, m->bytes, hipGetErrorString(e));
    }
    uint8_t *base = (uint8_t *)m->alloc;
    m->m.qs = base;
    m->m.tab = tab_bytes ? base + tab_at : nullptr;
    m->m.d = type == HQ_GGML_Q8_0 ? (const uint16_t *)(base + qbytes) : nullptr;
    std::lock_guard<std::mutex> lk(u->mu);
    auto fail_free = [&](hipError_t err) {
        (void)hipStreamSynchronize(u->st);
        (void)hipFree(m->alloc);
        free(m);
        return fail("%s: %s", who, hipGetErrorString(err));
    };
    if (type == HQ_GGML_Q8_0 && (e = hipMemsetAsync(base, 0, dev_bytes, u->st)) != hipSuccess) return fail_free(e);
    if (tab_bytes && (e = hipMemsetAsync(base + tab_at + tab_bytes, 0, HQ_Q4K_TAB_PAD, u->st)) != hipSuccess)
        return fail_free(e);
    const uint32_t rows_per = (uint32_t)(UP_CHUNK / rb < rows ? UP_CHUNK / rb : rows);
    bool used[2] = {false, false};
    for (uint32_t r0 = 0, i = 0; r0 < rows; r0 += rows_per, i++) {
        const int b = (int)(i & 1);
        const uint32_t n = rows - r0 < rows_per ? rows - r0 : rows_per;
        if (used[b] && (e = hipEventSynchronize(u->ev[b])) != hipSuccess) return fail_free(e);
        gather_rows(row_ptr, rb, r0, n, (uint8_t *)u->pinned[b]);
        const size_t bytes = (size_t)n * rb;
        if (!slot_bytes(type) && type != HQ_GGML_Q8_0) {  // Q4_K, Q5_K: the GGUF bytes in place
            e = hipMemcpyAsync(base + (size_t)r0 * rb, u->pinned[b], bytes, hipMemcpyHostToDevice, u->st);
        } else {
            e = hipMemcpyAsync(u->raw[b], u->pinned[b], bytes, hipMemcpyHostToDevice, u->st);
            if (e == hipSuccess && type == HQ_GGML_Q8_0) {
                k_repack_q8_0<<<up_grid((size_t)n * nb), 256, 0, u->st>>>((const uint8_t *)u->raw[b], n, (uint32_t)nb,
                                                                          (uint32_t)ldd, base + (size_t)r0 * K,
                                                                          (uint16_t *)(base + qbytes) + (size_t)r0 * ldd);
                e = hipGetLastError();
            } else if (e == hipSuccess) {
                const uint32_t in = block_bytes(type) / 2, outh = (uint32_t)(slot_bytes(type) / 2);
                k_repack_slots<<<up_grid((size_t)n * nb * outh), 256, 0, u->st>>>((const uint16_t *)u->raw[b], (size_t)n * nb, in,
                                                                                  outh, (uint16_t *)(base + (size_t)r0 * drb));
                e = hipGetLastError();
            }
        }
        if (e == hipSuccess) e = hipEventRecord(u->ev[b], u->st);
        if (e != hipSuccess) return fail_free(e);
        used[b] = true;
    }
    if (tab_bytes && (e = hq_launch_q4k_tables(&m->m, base + tab_at, u->st)) != hipSuccess) return fail_free(e);
    if ((e = hipStreamSynchronize(u->st)) != hipSuccess) return fail_free(e);
    *out = m;
    return 0;
}

extern "C" int hq_mat_upload(const hq_wmat_t *w, int device, hq_mat **out) {
    *out = nullptr;
    size_t rb;
    if (check_wmat(w, "hq_mat_upload", &rb)) return -1;
    const uint8_t *src = (const uint8_t *)w->data;
    auto row_ptr = [&](uint32_t r) { return src + (size_t)storage_row(w->rows, w->perm_heads, r) * rb; };
    return upload_rows(w->ggml_type, w->rows, w->cols, row_ptr, device, "hq_mat_upload", out);
}

extern "C" int hq_mat_upload_pair(const hq_wmat_t *gate, const hq_wmat_t *up, int device, hq_mat **out) {
    *out = nullptr;
    size_t rb, rbu;
    if (check_wmat(gate, "hq_mat_upload_pair", &rb) || check_wmat(up, "hq_mat_upload_pair", &rbu)) return -1;
    if (gate->ggml_type != up->ggml_type || gate->rows != up->rows || gate->cols != up->cols)
        return fail("hq_mat_upload_pair: gate (type %d, [%u, %u]) and up (type %d, [%u, %u]) differ", gate->ggml_type,
                    gate->rows, gate->cols, up->ggml_type, up->rows, up->cols);
    if (gate->rows % 8) return fail("hq_mat_upload_pair: %u rows is not a multiple of 8", gate->rows);
    if (gate->rows > (1u << 29)) return fail("hq_mat_upload_pair: %u rows too many", gate->rows);
    const uint8_t *g = (const uint8_t *)gate->data, *u = (const uint8_t *)up->data;
    auto row_ptr = [&](uint32_t r) {
        const uint32_t k = r / 16, e = r % 16;
        return e < 8 ? g + (size_t)storage_row(gate->rows, gate->perm_heads, 8 * k + e) * rb
                     : u + (size_t)storage_row(up->rows, up->perm_heads, 8 * k + e - 8) * rb;
    };
    if (upload_rows(gate->ggml_type, 2 * gate->rows, gate->cols, row_ptr, device, "hq_mat_upload_pair", out)) return -1;
    (*out)->pair = 1;
    return 0;
}

extern "C" void hq_mat_free(hq_mat *m) {
    if (!m) return;
    if (use_device(m->device) == 0) (void)hipFree(m->alloc);
    free(m);
}

const hq_dev_mat *hq_mat_dev(const hq_mat *m) { return &m->m; }
int hq_mat_device(const hq_mat *m) { return m->device; }

extern "C" int hq_mat_shape(const hq_mat *m, uint32_t *rows, uint32_t *cols, int *ggml_type) {
    if (!m) return fail("hq_mat_shape: no matrix");
    if (rows) *rows = m->m.rows;
    if (cols) *cols = m->m.cols;
    if (ggml_type) *ggml_type = m->m.type;
    return 0;
}

extern "C" size_t hq_mat_device_bytes(const hq_mat *m) { return m ? m->bytes : 0; }

extern "C" int hq_mat_download(const hq_mat *m, void *out, size_t nbytes) {
    if (!m || !out) return fail("hq_mat_download: null argument");
    const size_t rb = (size_t)(m->m.cols / block_values(m->m.type)) * block_bytes(m->m.type), total = rb * m->m.rows;
    if (nbytes < total) return fail("hq_mat_download: need %zu bytes, got %zu", total, nbytes);
    if (use_device(m->device)) return -1;
    const bool in_place = m->m.type != HQ_GGML_Q8_0 && !slot_bytes(m->m.type);
    const size_t copy = in_place ? total : m->bytes;  // (not the Q4_K column tables)
    std::vector<uint8_t> host(copy);
    HIPCK(hipMemcpy(host.data(), m->alloc, copy, hipMemcpyDeviceToHost));
    uint8_t *dst = (uint8_t *)out;
    if (in_place) {
        memcpy(dst, host.data(), total);
        return 0;
    }
    if (slot_bytes(m->m.type)) {
        const size_t nb = m->m.cols / 256, bb = block_bytes(m->m.type), sb = slot_bytes(m->m.type);
        for (uint32_t r = 0; r < m->m.rows; r++)
            for (size_t b = 0; b < nb; b++)
                memcpy(dst + (size_t)r * rb + bb * b, host.data() + (size_t)r * m->m.row_bytes + b * sb, bb);
        return 0;
    }
    const size_t K = m->m.cols, nb = K / 32, ldd = (size_t)m->m.ldd;
    const uint16_t *dpl = (const uint16_t *)(host.data() + round_up((size_t)m->m.rows * K, 256));
    for (uint32_t r = 0; r < m->m.rows; r++)
        for (size_t b = 0; b < nb; b++) {
            uint8_t *blk = dst + (size_t)r * rb + 34 * b;
            const uint16_t d = dpl[(size_t)r * ldd + b];
            blk[0] = (uint8_t)d, blk[1] = (uint8_t)(d >> 8);
            for (int j = 0; j < 32; j++) blk[2 + j] = host[(size_t)r * K + 32 * b + j] ^ 0x80u;
        }
    return 0;
}

// ------------------------------------------------------------------------------------ compute
static hipStream_t S(void *s) { return (hipStream_t)s; }

static int aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Library-owned device buffers, per (device, stream): staging for host-pointer entry points and
// the GEMM workspace. Work queued on one stream runs in order, so a stream's buffers are never used
// by two launches at once; calls on different streams (which may run concurrently) get different
// buffers. Grown on demand (hipMalloc), so the first call of a larger shape allocates: capture a
// call into a HIP graph only after an eager call of the same shape on the same stream.
namespace {
struct Staging {  // slots: 0 x fp32, 1 x fp16, 2 y fp32 (hq_matmul_host), 3 embedding ids, 4 readout ids,
                  // 5 GEMM partial tiles, 6 GEMM tile counters (kept zero), 7 activation sub-block sums,
                  // 8 fp32 gate/up product of the unfused hq_gemm_swiglu path
    void *buf[9] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    size_t cap[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
};
std::mutex g_staging_mu;
std::map<std::pair<int, void *>, Staging> g_staging;
std::map<int, int> g_n_cu;

// The slot's buffer of at least `bytes` for (device, stream); *grew = 1 when it was (re)allocated.
int staging(int device, void *stream, int slot, size_t bytes, void **p, int *grew = nullptr) {
    std::lock_guard<std::mutex> lk(g_staging_mu);
    Staging &s = g_staging[std::make_pair(device, stream)];
    if (grew) *grew = 0;
    if (s.cap[slot] < bytes) {
        if (s.buf[slot]) HIPCK(hipFree(s.buf[slot]));
        s.buf[slot] = nullptr;
        s.cap[slot] = 0;
        HIPCK(hipMalloc(&s.buf[slot], bytes));
        s.cap[slot] = bytes;
        if (grew) *grew = 1;
    }
    *p = s.buf[slot];
    return 0;
}

// Frees the buffers of every device's workspace for `stream` (its work has finished).
void staging_release(void *stream) {
    std::lock_guard<std::mutex> lk(g_staging_mu);
    for (auto it = g_staging.begin(); it != g_staging.end();) {
        if (it->first.second != stream) {
            ++it;
            continue;
        }
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != it->first.first) (void)hipSetDevice(it->first.first);
        for (void *b : it->second.buf)
            if (b) (void)hipFree(b);
        if (cur >= 0 && cur != it->first.first) (void)hipSetDevice(cur);
        it = g_staging.erase(it);
    }
}

int device_cus(int device, int *n_cu) {
    std::lock_guard<std::mutex> lk(g_staging_mu);
    int &v = g_n_cu[device];
    if (!v) {
        int x = 0;
        HIPCK(hipDeviceGetAttribute(&x, hipDeviceAttributeMultiprocessorCount, device));
        v = x > 0 ? x : 1;
    }
    *n_cu = v;
    return 0;
}

// GEMM workspace of an M-row hq_gemm on W's device and `stream`. A counter array that grows is
// zeroed once here, synchronously; the kernels leave every counter back at zero.
int gemm_work(const hq_mat *W, int M, void *stream, HqGemmWork *wk) {
    int n_cu;
    if (device_cus(W->device, &n_cu)) return -1;
    size_t pb, cb, sb;
    hq_gemm_work_bytes(&W->m, M, n_cu, &pb, &cb, &sb);
    void *part, *cnt, *sums = nullptr;
    int grew = 0;
    if (staging(W->device, stream, 5, pb, &part) || staging(W->device, stream, 6, cb, &cnt, &grew)) return -1;
    if (sb && staging(W->device, stream, 7, sb, &sums)) return -1;
    if (grew && cb) HIPCK(hipMemset(cnt, 0, cb));
    wk->partials = (float *)part;
    wk->counters = (int *)cnt;
    wk->sums = (uint16_t *)sums;
    wk->n_cu = n_cu;
    return 0;
}

// Rows of A per GEMM launch: the kernels address A through 32-bit buffer ranges and form a row's
// element offset (row * K, rows up to one tile past the last) in 32-bit signed arithmetic, so one
// launch keeps (rows + 128) * K below 2^31; a longer M is cut into launches of whole 128-row tiles
// (the reference cuts at 512 rows, src/cuda_backend.cu:866-875).
size_t gemm_rows_per_launch(size_t K) {
    const long r = (long)(((size_t)1 << 31) - 1) / (long)K - 128;
    return r >= 128 ? (size_t)r & ~(size_t)127 : r >= 1 ? (size_t)r : 1;
}
}  // namespace

extern "C" int hq_dequant_f32(const hq_mat *W, uint32_t row0, uint32_t nrows, float *out, void *stream) {
    if (!W || !out) return fail("hq_dequant_f32: null argument");
    if (row0 > W->m.rows || nrows > W->m.rows - row0)
        return fail("hq_dequant_f32: rows [%u, %u) outside [0, %u)", row0, row0 + nrows, W->m.rows);
    if (!aligned(out, 16)) return fail("hq_dequant_f32: output must be 16-byte aligned");
    if (nrows == 0) return 0;
    if (use_device(W->device)) return -1;
    HIPCK(hq_launch_dequant(&W->m, row0, nullptr, nrows, out, S(stream)));
    return 0;
}

extern "C" int hq_gemm(const hq_mat *W, const uint16_t *A, int M, void *C, int c_is_f32, int accumulate, void *stream) {
    if (!W || !A || !C) return fail("hq_gemm: null argument");
    if (M < 1 || M > (1 << 23)) return fail("hq_gemm: M = %d (1 .. 8388608)", M);
    if (!aligned(A, 16)) return fail("hq_gemm: A must be 16-byte aligned");
    if (!aligned(C, c_is_f32 ? 4 : 2)) return fail("hq_gemm: C is misaligned");
    if (use_device(W->device)) return -1;
    const size_t K = W->m.cols, N = W->m.rows, c_bytes = c_is_f32 ? 4 : 2, step = gemm_rows_per_launch(K);
    for (size_t m0 = 0; m0 < (size_t)M; m0 += step) {
        const int mc = (int)((size_t)M - m0 < step ? (size_t)M - m0 : step);
        const uint16_t *Ap = A + m0 * K;
        void *Cp = (char *)C + m0 * N * c_bytes;
        if (mc == 1) {
            HIPCK(hq_launch_gemv(&W->m, Ap, Cp, c_is_f32, accumulate, S(stream)));
            continue;
        }
        HqGemmWork wk;
        if (gemm_work(W, mc, stream, &wk)) return -1;
        HIPCK(hq_launch_gemm(&W->m, Ap, mc, Cp, c_is_f32, accumulate, wk, S(stream)));
    }
    return 0;
}

// ------------------------------------------------------------------------------------ no-alloc GEMM
// hq_gemm_noalloc's workspace: one file-scope device array per GPU (allocated with the code object,
// held until the process ends). Fixed layout: the per-tile counters first (HQ_NOALLOC_COUNTER_BYTES;
// only counter logic touches them, and every kernel leaves them at zero), then the partial tiles,
// then the activation sub-block sums. Host code never passes `scratch` itself to a kernel: its
// device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) unsigned char scratch[HQ_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
std::map<int, unsigned char *> g_scratch;  // device -> address of that device's `scratch`

__global__ void k_zero_words(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

// Address of `scratch` on `device` (the current device); the first call per device looks it up and
// zeroes the counter region with a fill kernel on `stream`, then waits for it.
int scratch_ptr(int device, void *stream, unsigned char **out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch.find(device);
    if (it != g_scratch.end()) {
        *out = it->second;
        return 0;
    }
    unsigned char *ptr = nullptr;
    HIPCK(hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch)));
    k_zero_words<<<64, 256, 0, S(stream)>>>((uint32_t *)ptr, HQ_NOALLOC_COUNTER_BYTES / 4);
    HIPCK(hipGetLastError());
    HIPCK(hipStreamSynchronize(S(stream)));
    g_scratch[device] = ptr;
    *out = ptr;
    return 0;
}

// Byte offsets of the partial tiles and the sums inside `scratch` for an M-row launch, and whether
// the launch's workspace fits.
struct NoallocLayout {
    size_t partials, sums, end;
    bool fits;
};
NoallocLayout noalloc_layout(size_t pb, size_t cb, size_t sb) {
    NoallocLayout L;
    L.partials = HQ_NOALLOC_COUNTER_BYTES;
    L.sums = round_up(L.partials + pb, 256);
    L.end = L.sums + sb;
    L.fits = cb <= HQ_NOALLOC_COUNTER_BYTES && L.end <= HQ_NOALLOC_SCRATCH_BYTES;
    return L;
}
}  // namespace

extern "C" int hq_gemm_workspace_bytes(int ggml_type, int M, uint32_t N, uint32_t K, int n_cu, size_t *partial_bytes,
                                       size_t *counter_bytes, size_t *sums_bytes, int *fits_noalloc) {
    if (!block_values(ggml_type)) return fail("hq_gemm_workspace_bytes: type %d (supported: %s)", ggml_type, SUPPORTED);
    if (M < 2 || N == 0 || K == 0 || K % block_values(ggml_type) || n_cu < 1)
        return fail("hq_gemm_workspace_bytes: M = %d, N = %u, K = %u, n_cu = %d", M, N, K, n_cu);
    if ((size_t)M > gemm_rows_per_launch(K))
        return fail("hq_gemm_workspace_bytes: M = %d is more than one launch (%zu rows at K = %u)", M,
                    gemm_rows_per_launch(K), K);
    hq_dev_mat W = {};
    W.type = ggml_type;
    W.rows = N;
    W.cols = K;
    // the upload's device layout: k-quant super-blocks in their aligned slots, the Q8_0 scale plane
    const size_t nb = K / block_values(ggml_type);
    W.row_bytes = nb * (slot_bytes(ggml_type) ? slot_bytes(ggml_type) : block_bytes(ggml_type));
    W.ldd = ggml_type == HQ_GGML_Q8_0 ? (int)round_up(K / 32, 8) : 0;
    size_t pb, cb, sb;
    hq_gemm_work_bytes(&W, M, n_cu, &pb, &cb, &sb);
    if (partial_bytes) *partial_bytes = pb;
    if (counter_bytes) *counter_bytes = cb;
    if (sums_bytes) *sums_bytes = sb;
    if (fits_noalloc) *fits_noalloc = noalloc_layout(pb, cb, sb).fits ? 1 : 0;
    return 0;
}

extern "C" int hq_gemm_noalloc(const hq_mat *W, const uint16_t *A, int M, void *C, int c_is_f32, int accumulate,
                               void *stream) {
    if (!W || !A || !C) return fail("hq_gemm_noalloc: null argument");
    if (M < 1 || M > (1 << 23)) return fail("hq_gemm_noalloc: M = %d (1 .. 8388608)", M);
    if (!aligned(A, 16)) return fail("hq_gemm_noalloc: A must be 16-byte aligned");
    if (!aligned(C, c_is_f32 ? 4 : 2)) return fail("hq_gemm_noalloc: C is misaligned");
    if (use_device(W->device)) return -1;
    int n_cu;
    if (device_cus(W->device, &n_cu)) return -1;
    const size_t K = W->m.cols, N = W->m.rows, c_bytes = c_is_f32 ? 4 : 2, step = gemm_rows_per_launch(K);
    // every launch's workspace is checked before the first one is queued
    for (size_t m0 = 0; m0 < (size_t)M; m0 += step) {
        const int mc = (int)((size_t)M - m0 < step ? (size_t)M - m0 : step);
        if (mc == 1) continue;
        size_t pb, cb, sb;
        hq_gemm_work_bytes(&W->m, mc, n_cu, &pb, &cb, &sb);
        const NoallocLayout L = noalloc_layout(pb, cb, sb);
        if (!L.fits)
            return fail("hq_gemm_noalloc: an M = %d launch needs %zu bytes of workspace (%zu of counters); the "
                        "preallocated scratch holds %d (%d of counters): use hq_gemm",
                        mc, L.end, cb, HQ_NOALLOC_SCRATCH_BYTES, HQ_NOALLOC_COUNTER_BYTES);
    }
    unsigned char *ptr;
    if (scratch_ptr(W->device, stream, &ptr)) return -1;
    for (size_t m0 = 0; m0 < (size_t)M; m0 += step) {
        const int mc = (int)((size_t)M - m0 < step ? (size_t)M - m0 : step);
        const uint16_t *Ap = A + m0 * K;
        void *Cp = (char *)C + m0 * N * c_bytes;
        if (mc == 1) {
            HIPCK(hq_launch_gemv(&W->m, Ap, Cp, c_is_f32, accumulate, S(stream)));
            continue;
        }
        size_t pb, cb, sb;
        hq_gemm_work_bytes(&W->m, mc, n_cu, &pb, &cb, &sb);
        const NoallocLayout L = noalloc_layout(pb, cb, sb);
        HqGemmWork wk;
        wk.counters = (int *)ptr;
        wk.partials = (float *)(ptr + L.partials);
        wk.sums = sb ? (uint16_t *)(ptr + L.sums) : nullptr;
        wk.n_cu = n_cu;
        HIPCK(hq_launch_gemm(&W->m, Ap, mc, Cp, c_is_f32, accumulate, wk, S(stream)));
    }
    return 0;
}

extern "C" int hq_gemv(const hq_mat *W, const uint16_t *a, void *c, int c_is_f32, int accumulate, void *stream) {
    return hq_gemm(W, a, 1, c, c_is_f32, accumulate, stream);
}

extern "C" int hq_gemm_swiglu(const hq_mat *pair, const uint16_t *A, int M, uint16_t *out, void *stream) {
    if (!pair || !A || !out) return fail("hq_gemm_swiglu: null argument");
    if (!pair->pair) return fail("hq_gemm_swiglu: not a gate/up pair matrix (hq_mat_upload_pair)");
    if (M < 1 || M > (1 << 23)) return fail("hq_gemm_swiglu: M = %d (1 .. 8388608)", M);
    if (!aligned(A, 16) || !aligned(out, 16)) return fail("hq_gemm_swiglu: A and out must be 16-byte aligned");
    if (use_device(pair->device)) return -1;
    const size_t K = pair->m.cols, N2 = pair->m.rows, step = gemm_rows_per_launch(K);
    for (size_t m0 = 0; m0 < (size_t)M; m0 += step) {
        const int mc = (int)((size_t)M - m0 < step ? (size_t)M - m0 : step);
        const uint16_t *Ap = A + m0 * K;
        uint16_t *Op = out + m0 * (N2 / 2);
        HqGemmWork wk = {};
        int fused = 0;
        if (mc > 1) {
            if (gemm_work(pair, mc, stream, &wk)) return -1;
            HIPCK(hq_launch_gemm_swiglu(&pair->m, Ap, mc, Op, wk, S(stream), &fused));
        }
        if (fused) continue;
        // other shapes: the product in fp32 (one pass over A for both halves), then the epilogue
        void *tmp;
        if (staging(pair->device, stream, 8, (size_t)mc * N2 * sizeof(float), &tmp)) return -1;
        if (mc == 1) {
            HIPCK(hq_launch_gemv(&pair->m, Ap, tmp, 1, 0, S(stream)));
        } else {
            HIPCK(hq_launch_gemm(&pair->m, Ap, mc, tmp, 1, 0, wk, S(stream)));
        }
        HIPCK(hq_launch_swiglu_pairs((const float *)tmp, Op, (size_t)mc * (N2 / 2), S(stream)));
    }
    return 0;
}

extern "C" int hq_gather_dot_dev(const hq_mat *head, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                                 void *stream) {
    if (!head || !H || !ids || !out) return fail("hq_gather_dot: null argument");
    if (B < 0 || k < 0 || (long)B * k > (1l << 30)) return fail("hq_gather_dot: B = %d, k = %d", B, k);
    if (!aligned(H, 16)) return fail("hq_gather_dot: H must be 16-byte aligned");
    if ((long)B * k == 0) return 0;
    if (use_device(head->device)) return -1;
    HIPCK(hq_launch_gather(&head->m, H, ids, B, k, out, S(stream)));
    return 0;
}


extern "C" int hq_gather_dot(const hq_mat *head, const uint16_t *H, const uint32_t *ids, int B, int k, float *out,
                             void *stream) {
    if (!head || !ids) return fail("hq_gather_dot: null argument");
    if (B < 0 || k < 0 || (long)B * k > (1l << 30)) return fail("hq_gather_dot: B = %d, k = %d", B, k);
    const size_t n = (size_t)B * k;
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= head->m.rows) return fail("hq_gather_dot: readout id %u out of range", ids[i]);
    if (n == 0) return 0;
    if (use_device(head->device)) return -1;
    void *d_ids;
    if (staging(head->device, stream, 4, n * sizeof(uint32_t), &d_ids)) return -1;
    HIPCK(hipMemcpyAsync(d_ids, ids, n * sizeof(uint32_t), hipMemcpyHostToDevice, S(stream)));
    return hq_gather_dot_dev(head, H, (const uint32_t *)d_ids, B, k, out, stream);
}

extern "C" int hq_embed_f32(const hq_mat *W, const uint32_t *ids, int n, float *out, void *stream) {
    if (!W || !ids || !out) return fail("hq_embed_f32: null argument");
    if (n < 0) return fail("hq_embed_f32: n = %d", n);
    for (int i = 0; i < n; i++)
        if (ids[i] >= W->m.rows) return fail("hq_embed_f32: token %u out of range", ids[i]);
    if (!aligned(out, 16)) return fail("hq_embed_f32: output must be 16-byte aligned");
    if (n == 0) return 0;
    if (use_device(W->device)) return -1;
    void *d_ids;
    if (staging(W->device, stream, 3, (size_t)n * sizeof(uint32_t), &d_ids)) return -1;
    HIPCK(hipMemcpyAsync(d_ids, ids, (size_t)n * sizeof(uint32_t), hipMemcpyHostToDevice, S(stream)));
    HIPCK(hq_launch_dequant(&W->m, 0, (const uint32_t *)d_ids, (uint32_t)n, out, S(stream)));
    return 0;
}

extern "C" int hq_matmul_host(const hq_mat *W, const float *x, size_t T, float *y, bool accumulate) {
    if (!W || !x || !y) return fail("hq_matmul_host: null argument");
    if (T == 0) return 0;
    if (T > (1u << 24)) return fail("hq_matmul_host: T = %zu", T);
    const size_t K = W->m.cols, N = W->m.rows;
    if (use_device(W->device)) return -1;
    void *dx, *dh, *dy;
    if (staging(W->device, nullptr, 0, T * K * sizeof(float), &dx) || staging(W->device, nullptr, 1, T * K * 2, &dh) ||
        staging(W->device, nullptr, 2, T * N * sizeof(float), &dy))
        return -1;
    HIPCK(hipMemcpy(dx, x, T * K * sizeof(float), hipMemcpyHostToDevice));
    if (accumulate) HIPCK(hipMemcpy(dy, y, T * N * sizeof(float), hipMemcpyHostToDevice));
    HIPCK(hq_launch_f32_to_f16((const float *)dx, (uint16_t *)dh, T * K, nullptr));
    if (hq_gemm(W, (const uint16_t *)dh, (int)T, dy, 1, accumulate ? 1 : 0, nullptr)) return -1;
    HIPCK(hipMemcpy(y, dy, T * N * sizeof(float), hipMemcpyDeviceToHost));
    return 0;
}

// ------------------------------------------------------------------------------------ plumbing
extern "C" int hq_malloc(void **p, size_t n) {
    HIPCK(hipMalloc(p, n ? n : 16));
    return 0;
}
extern "C" int hq_free(void *p) {
    HIPCK(hipFree(p));
    return 0;
}
extern "C" int hq_memcpy_h2d(void *dst, const void *src, size_t n, void *stream) {
    HIPCK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, S(stream)));
    HIPCK(hipStreamSynchronize(S(stream)));
    return 0;
}
extern "C" int hq_memcpy_d2d(void *dst, const void *src, size_t n, void *stream) {
    HIPCK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, S(stream)));
    return 0;
}

extern "C" int hq_memcpy_d2h(void *dst, const void *src, size_t n, void *stream) {
    HIPCK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, S(stream)));
    HIPCK(hipStreamSynchronize(S(stream)));
    return 0;
}
extern "C" int hq_memset(void *dst, int value, size_t n, void *stream) {
    HIPCK(hipMemsetAsync(dst, value, n, S(stream)));
    return 0;
}
extern "C" int hq_stream_create(void **stream) {
    hipStream_t s;
    HIPCK(hipStreamCreate(&s));
    *stream = (void *)s;
    return 0;
}
extern "C" int hq_stream_destroy(void *stream) {
    HIPCK(hipStreamSynchronize(S(stream)));
    staging_release(stream);  // the stream's workspace: a later stream may get the same handle
    HIPCK(hipStreamDestroy(S(stream)));
    return 0;
}
extern "C" int hq_stream_synchronize(void *stream) {
    HIPCK(hipStreamSynchronize(S(stream)));
    return 0;
}
extern "C" int hq_device_synchronize(void) {
    HIPCK(hipDeviceSynchronize());
    return 0;
}

extern "C" void hq_gemm_kernel(int ggml_type, int M, int N, int K, char *name, int name_bytes) {
    if (!name || name_bytes <= 0) return;
    hq_gemm_kernel_name(ggml_type, M, N, K, 256, name, (size_t)name_bytes);
}

extern "C" void hq_gemm_tiles(int ggml_type, int M, int N, int *rows_per_tile, int *cols_per_tile) {
    (void)N;
    int r = 1, c = 16;
    if (M > 1) hq_gemm_tile_shape(ggml_type, M, N, 256, 256, &r, &c);
    if (rows_per_tile) *rows_per_tile = r;
    if (cols_per_tile) *cols_per_tile = c;
}

// ------------------------------------------------------------------------------------ timing
namespace {
template <typename F>
int time_graph(int iters, int reps, void *stream, float *ms, F launch) {
    if (iters < 1 || reps < 1 || reps > 64) return fail("hq_time: iters = %d, reps = %d (1 .. 64)", iters, reps);
    if (!stream) return fail("hq_time: needs a created stream (graph capture)");
    hipStream_t st = S(stream);
    // replay r is its own graph of launches r * iters .. r * iters + iters - 1, so that launches keep
    // rotating over the caller's buffers across replays
    std::vector<hipGraph_t> g(reps, nullptr);
    std::vector<hipGraphExec_t> ge(reps, nullptr);
    std::vector<hipEvent_t> ev(reps + 1, nullptr);
    auto cleanup = [&]() {
        for (auto &x : ev)
            if (x) (void)hipEventDestroy(x);
        for (auto &x : ge)
            if (x) (void)hipGraphExecDestroy(x);
        for (auto &x : g)
            if (x) (void)hipGraphDestroy(x);
    };
    for (int r = 0; r < reps; r++) {
        hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) {
            cleanup();
            return fail("hipStreamBeginCapture: %s", hipGetErrorString(e));
        }
        int rc = 0;
        for (int i = 0; i < iters && !rc; i++) rc = launch(r * iters + i);
        e = hipStreamEndCapture(st, &g[r]);
        if (rc) {
            cleanup();
            return -1;
        }
        if (e == hipSuccess) e = hipGraphInstantiate(&ge[r], g[r], nullptr, nullptr, 0);
        if (e != hipSuccess) {
            cleanup();
            return fail("graph capture: %s", hipGetErrorString(e));
        }
    }
    // one event between consecutive replays: replay r's time is ev[r] .. ev[r + 1]; the result is the
    // median over the replays of the time per launch
    hipError_t e = hipSuccess;
    for (auto &x : ev)
        if (e == hipSuccess) e = hipEventCreate(&x);
    if (e == hipSuccess) e = hipGraphLaunch(ge[reps - 1], st);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(ev[0], st);
    for (int r = 0; r < reps && e == hipSuccess; r++) {
        e = hipGraphLaunch(ge[r], st);
        if (e == hipSuccess) e = hipEventRecord(ev[r + 1], st);
    }
    if (e == hipSuccess) e = hipEventSynchronize(ev[reps]);
    std::vector<float> per(reps);
    for (int r = 0; r < reps && e == hipSuccess; r++) {
        e = hipEventElapsedTime(&per[r], ev[r], ev[r + 1]);
        per[r] /= (float)iters;
    }
    cleanup();
    if (e != hipSuccess) return fail("hq_time: %s", hipGetErrorString(e));
    std::sort(per.begin(), per.end());
    *ms = reps % 2 ? per[reps / 2] : 0.5f * (per[reps / 2 - 1] + per[reps / 2]);
    return 0;
}
}  // namespace

extern "C" int hq_time_gemm(hq_mat *const *Ws, int n_w, const uint16_t *A, int M, void *C, int c_is_f32, int iters,
                            int reps, void *stream, float *ms) {
    if (!Ws || n_w < 1) return fail("hq_time_gemm: no matrices");
    for (int i = 0; i < n_w; i++)
        if (!Ws[i] || Ws[i]->m.rows != Ws[0]->m.rows || Ws[i]->m.cols != Ws[0]->m.cols || Ws[i]->m.type != Ws[0]->m.type)
            return fail("hq_time_gemm: matrices differ in shape or type");
    if (hq_gemm(Ws[0], A, M, C, c_is_f32, 0, stream)) return -1;  // sizes the workspace outside the capture
    HIPCK(hipStreamSynchronize(S(stream)));
    return time_graph(iters, reps, stream, ms,
                      [&](int i) { return hq_gemm(Ws[i % n_w], A, M, C, c_is_f32, 0, stream); });
}

extern "C" int hq_time_gemm_kernel(hq_mat *const *Ws, int n_w, const uint16_t *A, int M, void *C, int c_is_f32,
                                   int iters, int reps, void *stream, float *ms) {
    if (!Ws || n_w < 1) return fail("hq_time_gemm_kernel: no matrices");
    if (M < 2) return fail("hq_time_gemm_kernel: M = %d (the GEMM kernels run for M >= 2)", M);
    for (int i = 0; i < n_w; i++)
        if (!Ws[i] || Ws[i]->m.rows != Ws[0]->m.rows || Ws[i]->m.cols != Ws[0]->m.cols || Ws[i]->m.type != Ws[0]->m.type)
            return fail("hq_time_gemm_kernel: matrices differ in shape or type");
    if (!aligned(A, 16)) return fail("hq_time_gemm_kernel: A must be 16-byte aligned");
    if (use_device(Ws[0]->device)) return -1;
    HqGemmWork wk;
    if ((size_t)M > gemm_rows_per_launch(Ws[0]->m.cols))
        return fail("hq_time_gemm_kernel: M = %d exceeds one launch's %zu rows at K = %u", M,
                    gemm_rows_per_launch(Ws[0]->m.cols), Ws[0]->m.cols);
    if (gemm_work(Ws[0], M, stream, &wk)) return -1;
    // the pre-pass depends on A only: run it once, then time the main kernel alone
    HIPCK(hq_launch_gemm_pre(&Ws[0]->m, A, M, wk, S(stream)));
    HIPCK(hq_launch_gemm_main(&Ws[0]->m, A, M, C, c_is_f32, 0, wk, S(stream)));
    HIPCK(hipStreamSynchronize(S(stream)));
    return time_graph(iters, reps, stream, ms, [&](int i) {
        HIPCK(hq_launch_gemm_main(&Ws[i % n_w]->m, A, M, C, c_is_f32, 0, wk, S(stream)));
        return 0;
    });
}

extern "C" int hq_time_gemm_swiglu(hq_mat *const *pairs, int n_w, const uint16_t *A, int M, uint16_t *out, int iters,
                                   int reps, void *stream, float *ms) {
    if (!pairs || n_w < 1) return fail("hq_time_gemm_swiglu: no matrices");
    for (int i = 0; i < n_w; i++)
        if (!pairs[i] || pairs[i]->m.rows != pairs[0]->m.rows || pairs[i]->m.cols != pairs[0]->m.cols ||
            pairs[i]->m.type != pairs[0]->m.type)
            return fail("hq_time_gemm_swiglu: matrices differ in shape or type");
    if (hq_gemm_swiglu(pairs[0], A, M, out, stream)) return -1;  // sizes the workspace outside the capture
    HIPCK(hipStreamSynchronize(S(stream)));
    return time_graph(iters, reps, stream, ms, [&](int i) { return hq_gemm_swiglu(pairs[i % n_w], A, M, out, stream); });
}

extern "C" int hq_time_read(void *const *bufs, int n_bufs, size_t bytes, int grid, int iters, int reps, void *stream,
                            float *ms) {
    if (!bufs || n_bufs < 1 || bytes == 0 || bytes % 16) return fail("hq_time_read: %d buffers of %zu bytes", n_bufs, bytes);
    if (grid < 1 || grid > (1 << 20)) return fail("hq_time_read: grid %d", grid);
    for (int i = 0; i < n_bufs; i++)
        if (!bufs[i] || !aligned(bufs[i], 16)) return fail("hq_time_read: buffer %d missing or not 16-byte aligned", i);
    int dev;
    HIPCK(hipGetDevice(&dev));
    void *out;
    if (staging(dev, stream, 3, (size_t)grid * 16, &out)) return -1;  // (outside the capture)
    HIPCK(hipStreamSynchronize(S(stream)));
    return time_graph(iters, reps, stream, ms, [&](int i) {
        const hipError_t e = hq_launch_stream_read(bufs[i % n_bufs], bytes, (uint32_t *)out, (unsigned)grid, S(stream));
        return e == hipSuccess ? 0 : fail("hq_time_read: %s", hipGetErrorString(e));
    });
}

extern "C" int hq_time_gather(hq_mat *const *Ws, int n_w, const uint16_t *H, const uint32_t *ids_dev, int n_sets,
                              int B, int k, float *out, int iters, int reps, void *stream, float *ms) {
    if (!Ws || n_w < 1) return fail("hq_time_gather: no matrices");
    if (n_sets < 1) return fail("hq_time_gather: n_sets = %d", n_sets);
    for (int i = 0; i < n_w; i++)
        if (!Ws[i] || Ws[i]->m.rows != Ws[0]->m.rows || Ws[i]->m.cols != Ws[0]->m.cols || Ws[i]->m.type != Ws[0]->m.type)
            return fail("hq_time_gather: matrices differ in shape or type");
    return time_graph(iters, reps, stream, ms,
                      [&](int i) {
                          return hq_gather_dot_dev(Ws[i % n_w], H, ids_dev + (size_t)(i % n_sets) * B * k, B, k, out,
                                                   stream);
                      });
}
