// ssm_file.hip — .ssm weight files: the validating reader, the HBM upload, the
// model's weight lookups, a streaming writer, the exporter's quantizer and a
// random-init model writer.  Host code only.
//
// The format is the reference's (include/lite_ssm/ssm_format.hpp): a 96-byte
// header, index entries of a 32-byte prefix + u64 shape[rank] + name padded to
// 8 bytes, then payloads at 64-byte aligned absolute offsets.  Codes 7 and 8
// (Q4_G64, Q8_G32) extend the dtype list with the INT4_B32 layout rule.
//
// Upload: the reference wraps the mmap in a shared MTLBuffer (no copy,
// metal_buffer.mm:37-67).  On MI355X the weights must live in HBM, so the file
// is copied once: the mapping is read into two pinned staging buffers by a few
// host threads while the other buffer's DMA to the device runs, which keeps the
// link busy without registering the mapping itself.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "internal.hpp"

using namespace lssm;

namespace {

constexpr char kMagic[4] = {'L', 'S', 'S', 'M'};
constexpr uint32_t kVersion = 1;
constexpr uint64_t kDataAlign = 64;
constexpr uint32_t kMaxRank = LSSM_SSM_MAX_RANK;

// On-disk header, byte for byte (ssm_format.hpp:73-110).
#pragma pack(push, 1)
struct DiskHeader {
    char magic[4];
    uint32_t version, header_size, n_tensors;
    uint64_t index_offset, data_offset;
    uint32_t d_model, n_layer, d_state, d_conv, expand, vocab_size;
    uint32_t n_heads, d_head, chunk_size, default_dtype, n_groups, norm_before_gate;
    uint32_t reserved[4];
};
struct DiskEntry {            // fixed prefix of one index entry (ssm_format.hpp:117-124)
    uint32_t name_len, rank, dtype, pad0;
    uint64_t offset, nbytes;
};
#pragma pack(pop)
static_assert(sizeof(DiskHeader) == 96, "header layout");
static_assert(sizeof(DiskEntry) == 32, "index entry layout");

inline uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

uint64_t packed_nbytes(uint32_t dt, uint64_t numel) {
    switch (dt) {
        case LSSM_DTYPE_F16: case LSSM_DTYPE_BF16: return numel * 2;
        case LSSM_DTYPE_F32: case LSSM_DTYPE_I32: return numel * 4;
        case LSSM_DTYPE_I8: case LSSM_DTYPE_U8: return numel;
        case LSSM_DTYPE_INT4_B32: return numel / 2 + numel / 32 * 2;
        case LSSM_DTYPE_Q4_G64: return numel / 2 + numel / 64 * 2;
        case LSSM_DTYPE_Q8_G32: return numel + numel / 32 * 2;
        default: return 0;
    }
}

// numel of a shape, false on u64 overflow
bool shape_numel(const uint64_t* shape, uint32_t rank, uint64_t* out) {
    uint64_t n = 1;
    for (uint32_t i = 0; i < rank; ++i)
        if (__builtin_mul_overflow(n, shape[i], &n)) return false;
    *out = n;
    return true;
}

struct Entry {
    std::string name;
    lssm_ssm_tensor t{};
};

}  // namespace

struct lssm_ssm {
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    DiskHeader hdr{};
    std::vector<Entry> entries;                      // file order
    std::unordered_map<std::string, size_t> by_name;
    void* dev = nullptr;                             // HBM copy of the whole file
    int dev_id = -1;
};

namespace {

int parse(lssm_ssm* f) {
    const uint8_t* base = f->base;
    const uint64_t size = f->size;
    // [pos, pos + n) inside the file
    auto in_bounds = [&](uint64_t pos, uint64_t n) { return pos <= size && n <= size - pos; };
    if (size < sizeof(DiskHeader))
        return set_error(LSSM_EINVAL, "SSMFile: file too small to contain a header (%llu bytes)",
                         (unsigned long long)size);
    DiskHeader& h = f->hdr;
    std::memcpy(&h, base, sizeof(h));
    if (std::memcmp(h.magic, kMagic, 4) != 0)
        return set_error(LSSM_EINVAL, "SSMFile: bad magic; not a .ssm file");
    if (h.version != kVersion)
        return set_error(LSSM_EINVAL, "SSMFile: unsupported version %u (expected %u)", h.version,
                         kVersion);
    if (h.header_size != sizeof(DiskHeader))
        return set_error(LSSM_EINVAL,
                         "SSMFile: header_size mismatch — file claims %u bytes, build expects %zu",
                         h.header_size, sizeof(DiskHeader));
    if (h.index_offset < sizeof(DiskHeader) || h.index_offset > size ||
        h.data_offset < h.index_offset || h.data_offset > size)
        return set_error(LSSM_EINVAL, "SSMFile: index/data offsets out of range");

    uint64_t pos = h.index_offset;
    f->entries.reserve(std::min<uint64_t>(h.n_tensors, size / sizeof(DiskEntry)));
    for (uint32_t i = 0; i < h.n_tensors; ++i) {
        if (!in_bounds(pos, sizeof(DiskEntry)))
            return set_error(LSSM_EINVAL, "SSMFile: out-of-bounds read while parsing tensor index prefix");
        DiskEntry e;
        std::memcpy(&e, base + pos, sizeof(e));
        pos += sizeof(e);
        if (e.rank == 0 || e.rank > kMaxRank)
            return set_error(LSSM_EINVAL, "SSMFile: tensor %u has unsupported rank %u", i, e.rank);
        const uint64_t shape_bytes = 8ull * e.rank;
        if (!in_bounds(pos, shape_bytes))
            return set_error(LSSM_EINVAL, "SSMFile: out-of-bounds read while parsing tensor shape");
        Entry ent;
        ent.t.dtype = e.dtype;
        ent.t.rank = e.rank;
        std::memcpy(ent.t.shape, base + pos, shape_bytes);
        pos += shape_bytes;
        if (!in_bounds(pos, e.name_len))
            return set_error(LSSM_EINVAL, "SSMFile: out-of-bounds read while parsing tensor name");
        ent.name.assign(reinterpret_cast<const char*>(base + pos), e.name_len);
        pos += e.name_len;
        const uint64_t raw = sizeof(DiskEntry) + shape_bytes + e.name_len;
        pos += round_up(raw, 8) - raw;   // entries are padded to 8 bytes

        if (e.offset > size || e.nbytes > size - e.offset)
            return set_error(LSSM_EINVAL, "SSMFile: payload for '%s' overflows file", ent.name.c_str());
        uint64_t numel = 0;
        if (!shape_numel(ent.t.shape, e.rank, &numel))
            return set_error(LSSM_EINVAL, "SSMFile: '%s' shape overflows", ent.name.c_str());
        const uint64_t expected = packed_nbytes(e.dtype, numel);
        if (expected != e.nbytes)
            return set_error(LSSM_EINVAL, "SSMFile: '%s' nbytes=%llu but expected packed=%llu",
                             ent.name.c_str(), (unsigned long long)e.nbytes,
                             (unsigned long long)expected);
        ent.t.offset = e.offset;
        ent.t.nbytes = e.nbytes;
        ent.t.host = base + e.offset;
        if (!f->by_name.emplace(ent.name, f->entries.size()).second)
            return set_error(LSSM_EINVAL, "SSMFile: duplicate tensor name in index");
        f->entries.push_back(std::move(ent));
        if (pos > h.data_offset)
            return set_error(LSSM_EINVAL, "SSMFile: index walk overran data_offset");
    }
    return LSSM_OK;
}

void release(lssm_ssm* f) {
    if (f->dev) {
        int cur = 0;
        if (hipGetDevice(&cur) == hipSuccess && cur != f->dev_id) (void)hipSetDevice(f->dev_id);
        (void)hipFree(f->dev);
        if (cur != f->dev_id) (void)hipSetDevice(cur);
    }
    if (f->base) munmap(const_cast<uint8_t*>(f->base), f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

const Entry* lookup(const lssm_ssm* f, const std::string& name) {
    auto it = f->by_name.find(name);
    return it == f->by_name.end() ? nullptr : &f->entries[it->second];
}

// Parallel copy of [src, src+n) into dst by up to `nt` threads.
void par_copy(void* dst, const void* src, size_t n, unsigned nt) {
    const size_t min_part = size_t(4) << 20;
    nt = std::max(1u, std::min<unsigned>(nt, unsigned((n + min_part - 1) / min_part)));
    if (nt == 1) {
        std::memcpy(dst, src, n);
        return;
    }
    std::vector<std::thread> th;
    const size_t part = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t lo = t * part, hi = std::min(n, lo + part);
        if (lo >= hi) break;
        th.emplace_back([=] {
            std::memcpy(static_cast<uint8_t*>(dst) + lo, static_cast<const uint8_t*>(src) + lo, hi - lo);
        });
    }
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" {

uint64_t lssm_ssm_packed_nbytes(uint32_t dtype, uint64_t numel) { return packed_nbytes(dtype, numel); }

int lssm_ssm_open(lssm_ssm** out, const char* path) {
    clear_error();
    if (!out || !path) return set_error(LSSM_EINVAL, "lssm_ssm_open: null argument");
    *out = nullptr;
    auto* f = new lssm_ssm();
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) {
        const int err = errno;
        release(f);
        return set_error(LSSM_EDEVICE, "MmapFile: open('%s') failed: %s", path, strerror(err));
    }
    struct stat st;
    if (fstat(f->fd, &st) != 0) {
        const int err = errno;
        release(f);
        return set_error(LSSM_EDEVICE, "MmapFile: fstat('%s') failed: %s", path, strerror(err));
    }
    f->size = static_cast<uint64_t>(st.st_size);
    if (f->size > 0) {
        void* p = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
        if (p == MAP_FAILED) {
            const int err = errno;
            f->size = 0;
            release(f);
            return set_error(LSSM_EDEVICE, "MmapFile: mmap('%s') failed: %s", path, strerror(err));
        }
        f->base = static_cast<const uint8_t*>(p);
    }
    const int rc = parse(f);
    if (rc != LSSM_OK) {
        release(f);
        return rc;
    }
    *out = f;
    return LSSM_OK;
}

int lssm_ssm_close(lssm_ssm* f) {
    clear_error();
    if (f) release(f);
    return LSSM_OK;
}

int lssm_ssm_get_header(const lssm_ssm* f, lssm_ssm_header* h) {
    clear_error();
    if (!f || !h) return set_error(LSSM_EINVAL, "lssm_ssm_get_header: null argument");
    const DiskHeader& d = f->hdr;
    *h = lssm_ssm_header{d.version, d.header_size, d.n_tensors, d.index_offset, d.data_offset,
                         f->size, d.d_model, d.n_layer, d.d_state, d.d_conv, d.expand,
                         d.vocab_size, d.n_heads, d.d_head, d.chunk_size, d.default_dtype,
                         d.n_groups == 0 ? 1u : d.n_groups, d.norm_before_gate};
    return LSSM_OK;
}

int lssm_ssm_tensor_at(const lssm_ssm* f, uint32_t i, char* name, size_t name_cap,
                       lssm_ssm_tensor* t) {
    clear_error();
    if (!f) return set_error(LSSM_EINVAL, "lssm_ssm_tensor_at: null file");
    if (i >= f->entries.size())
        return set_error(LSSM_EINVAL, "lssm_ssm_tensor_at: index %u out of range (%zu tensors)", i,
                         f->entries.size());
    const Entry& e = f->entries[i];
    if (name) {
        if (name_cap < e.name.size() + 1)
            return set_error(LSSM_EINVAL, "lssm_ssm_tensor_at: name needs %zu bytes", e.name.size() + 1);
        std::memcpy(name, e.name.c_str(), e.name.size() + 1);
    }
    if (t) *t = e.t;
    return LSSM_OK;
}

int lssm_ssm_find(const lssm_ssm* f, const char* name, lssm_ssm_tensor* t) {
    clear_error();
    if (!f || !name) return set_error(LSSM_EINVAL, "lssm_ssm_find: null argument");
    const Entry* e = lookup(f, name);
    if (!e) return set_error(LSSM_ENOTFOUND, "SSMFile: no tensor named '%s'", name);
    if (t) *t = e->t;
    return LSSM_OK;
}

int lssm_ssm_upload(lssm_ssm* f, lssm_ctx* ctx, void** device_base) {
    LSSM_CHECK_CTX(ctx);
    if (!f || !device_base) return set_error(LSSM_EINVAL, "lssm_ssm_upload: null argument");
    if (f->dev) {
        *device_base = f->dev;
        return LSSM_OK;
    }
    *device_base = nullptr;
    void* dev = nullptr;
    hipError_t e = hipMalloc(&dev, std::max<uint64_t>(f->size, 1));
    if (e != hipSuccess)
        return set_error(LSSM_EDEVICE, "UnifiedBuffer: hipMalloc(%llu): %s",
                         (unsigned long long)f->size, hipGetErrorString(e));
    constexpr size_t kChunk = size_t(64) << 20;
    const size_t chunk = std::min<size_t>(kChunk, std::max<uint64_t>(f->size, 1));
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    const unsigned nt = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    auto fail = [&](const char* what, hipError_t err) {
        (void)hipStreamSynchronize(ctx->stream);
        for (int b = 0; b < 2; ++b) {
            if (done[b]) (void)hipEventDestroy(done[b]);
            if (stage[b]) (void)hipHostFree(stage[b]);
        }
        (void)hipFree(dev);
        return set_error(LSSM_EDEVICE, "UnifiedBuffer: %s: %s", what, hipGetErrorString(err));
    };
    for (int b = 0; b < 2; ++b) {
        if ((e = hipHostMalloc(&stage[b], chunk, hipHostMallocDefault)) != hipSuccess)
            return fail("hipHostMalloc", e);
        if ((e = hipEventCreateWithFlags(&done[b], hipEventDisableTiming)) != hipSuccess)
            return fail("hipEventCreate", e);
    }
    uint64_t off = 0;
    for (int k = 0; off < f->size; ++k, off += chunk) {
        const int b = k & 1;
        const size_t n = std::min<uint64_t>(chunk, f->size - off);
        if (used[b] && (e = hipEventSynchronize(done[b])) != hipSuccess) return fail("staging wait", e);
        par_copy(stage[b], f->base + off, n, nt);
        if ((e = hipMemcpyAsync(static_cast<uint8_t*>(dev) + off, stage[b], n, hipMemcpyHostToDevice,
                                ctx->stream)) != hipSuccess)
            return fail("hipMemcpyAsync", e);
        if ((e = hipEventRecord(done[b], ctx->stream)) != hipSuccess) return fail("hipEventRecord", e);
        used[b] = true;
    }
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return fail("hipStreamSynchronize", e);
    for (int b = 0; b < 2; ++b) {
        (void)hipEventDestroy(done[b]);
        (void)hipHostFree(stage[b]);
    }
    (void)hipGetDevice(&f->dev_id);
    f->dev = dev;
    *device_base = dev;
    return LSSM_OK;
}

int lssm_ssm_model(const lssm_ssm* f, const void* device_base, lssm_model_config* cfg,
                   const void** embed, const void** norm_f, const void** lm_head,
                   lssm_layer_weights* layers, uint32_t n_layers_cap) {
    clear_error();
    if (!f || !cfg || !embed || !norm_f || !lm_head || !layers)
        return set_error(LSSM_EINVAL, "lssm_ssm_model: null argument");
    if (!device_base) return set_error(LSSM_EINVAL, "Mamba2Model: SSMFile missing buffer or mmap");
    const DiskHeader& h = f->hdr;
    lssm_model_config c{};
    c.d_model = h.d_model; c.n_layer = h.n_layer; c.d_state = h.d_state; c.d_conv = h.d_conv;
    c.expand = h.expand; c.vocab_size = h.vocab_size; c.n_heads = h.n_heads; c.d_head = h.d_head;
    c.chunk_size = h.chunk_size; c.n_groups = h.n_groups == 0 ? 1u : h.n_groups;
    LSSM_REQUIRE(c.n_layer <= n_layers_cap, "lssm_ssm_model: file has %u layers, room for %u",
                 c.n_layer, n_layers_cap);
    const uint64_t d_inner = uint64_t(c.expand) * c.d_model;
    const uint64_t xbc = d_inner + 2ull * c.n_groups * c.d_state;
    const uint64_t proj = d_inner + xbc + c.n_heads;
    LSSM_REQUIRE(c.d_model && c.n_layer && c.n_heads && c.d_head && c.vocab_size && c.d_conv,
                 "Mamba2Model: zero dimension in the file header");
    LSSM_REQUIRE(uint64_t(c.n_heads) * c.d_head == d_inner,
                 "Mamba2Model: n_heads * d_head (%u * %u) != expand * d_model (%llu)", c.n_heads,
                 c.d_head, (unsigned long long)d_inner);

    auto find = [&](const std::string& name, const Entry** out) -> int {
        *out = lookup(f, name);
        if (!*out) return set_error(LSSM_EINVAL, "Mamba2Model: missing tensor '%s'", name.c_str());
        return LSSM_OK;
    };
    auto numel = [](const Entry* e) {
        uint64_t n = 1;
        for (uint32_t i = 0; i < e->t.rank; ++i) n *= e->t.shape[i];
        return n;
    };
    auto dev = [&](const Entry* e) -> const void* {
        return static_cast<const uint8_t*>(device_base) + e->t.offset;
    };

    const Entry* nf;
    if (int rc = find("backbone.norm_f.weight", &nf)) return rc;
    const uint32_t act = nf->t.dtype;
    LSSM_REQUIRE(act == LSSM_DTYPE_F16 || act == LSSM_DTYPE_BF16 || act == LSSM_DTYPE_F32,
                 "Mamba2Model: backbone.norm_f.weight has dtype %u; activations must be f16, bf16 or f32",
                 act);
    c.act = act;
    // a tensor of the activation dtype with exactly `n` elements
    auto plain = [&](const Entry* e, uint64_t n) -> int {
        if (e->t.dtype != act)
            return set_error(LSSM_EINVAL, "Mamba2Model: '%s' has dtype %u, expected %u (that of norm_f)",
                             e->name.c_str(), e->t.dtype, act);
        if (numel(e) != n)
            return set_error(LSSM_EINVAL, "Mamba2Model: '%s' has %llu elements, expected %llu",
                             e->name.c_str(), (unsigned long long)numel(e), (unsigned long long)n);
        return LSSM_OK;
    };
    if (int rc = plain(nf, c.d_model)) return rc;

    const Entry* emb;
    if (int rc = find("backbone.embeddings.weight", &emb)) return rc;
    LSSM_REQUIRE(emb->t.rank == 2 && emb->t.shape[1] == c.d_model && emb->t.shape[0] >= c.vocab_size &&
                 emb->t.dtype == act,
                 "Mamba2Model: backbone.embeddings.weight must be [>= vocab_size %u, d_model %u] of "
                 "dtype %u", c.vocab_size, c.d_model, act);
    const Entry* head = lookup(f, "lm_head.weight");
    if (head)
        LSSM_REQUIRE(head->t.rank == 2 && head->t.shape[1] == c.d_model &&
                     head->t.shape[0] >= c.vocab_size && head->t.dtype == act,
                     "Mamba2Model: lm_head.weight must be [>= vocab_size %u, d_model %u] of dtype %u",
                     c.vocab_size, c.d_model, act);
    else
        head = emb;

    int wdt = -1;
    for (uint32_t i = 0; i < c.n_layer; ++i) {
        const std::string p = "backbone.layers." + std::to_string(i) + ".";
        const Entry *nw, *ip, *cw, *cb, *dtb, *al, *dd, *mn, *op;
        if (int rc = find(p + "norm.weight", &nw)) return rc;
        if (int rc = find(p + "mixer.in_proj.weight", &ip)) return rc;
        if (int rc = find(p + "mixer.conv1d.weight", &cw)) return rc;
        if (int rc = find(p + "mixer.conv1d.bias", &cb)) return rc;
        if (int rc = find(p + "mixer.dt_bias", &dtb)) return rc;
        if (int rc = find(p + "mixer.A_log", &al)) return rc;
        if (int rc = find(p + "mixer.D", &dd)) return rc;
        if (int rc = find(p + "mixer.norm.weight", &mn)) return rc;
        if (int rc = find(p + "mixer.out_proj.weight", &op)) return rc;

        if (ip->t.rank != 2 || ip->t.shape[0] != proj)
            return set_error(LSSM_EINVAL,
                             "Mamba2Model: in_proj output dim mismatch vs config (got %llu, expected %llu)",
                             (unsigned long long)ip->t.shape[0], (unsigned long long)proj);
        if (cw->t.shape[0] != xbc)
            return set_error(LSSM_EINVAL, "Mamba2Model: conv1d weight dim mismatch vs config");
        LSSM_REQUIRE(ip->t.shape[1] == c.d_model, "Mamba2Model: '%s' must have d_model (%u) columns",
                     ip->name.c_str(), c.d_model);
        LSSM_REQUIRE(op->t.rank == 2 && op->t.shape[0] == c.d_model && op->t.shape[1] == d_inner,
                     "Mamba2Model: '%s' must be [d_model %u, d_inner %llu]", op->name.c_str(),
                     c.d_model, (unsigned long long)d_inner);
        // in_proj and out_proj share one format across the model
        const int dt_ip = static_cast<int>(ip->t.dtype);
        if (wdt < 0) wdt = dt_ip;
        LSSM_REQUIRE(dt_ip == wdt && static_cast<int>(op->t.dtype) == wdt,
                     "Mamba2Model: '%s' / '%s' have dtypes %u / %u; every in_proj and out_proj must "
                     "use the format of layer 0's in_proj (%d)", ip->name.c_str(), op->name.c_str(),
                     ip->t.dtype, op->t.dtype, wdt);
        if (int rc = plain(nw, c.d_model)) return rc;
        if (int rc = plain(cw, xbc * c.d_conv)) return rc;
        if (int rc = plain(cb, xbc)) return rc;
        if (int rc = plain(dtb, c.n_heads)) return rc;
        if (int rc = plain(al, c.n_heads)) return rc;
        if (int rc = plain(dd, c.n_heads)) return rc;
        if (int rc = plain(mn, d_inner)) return rc;

        lssm_layer_weights& L = layers[i];
        L = lssm_layer_weights{};
        L.norm_w = dev(nw);
        L.conv1d_w = dev(cw);
        L.conv1d_b = dev(cb);
        L.dt_bias = dev(dtb);
        L.A_log = dev(al);
        L.D = dev(dd);
        L.mixer_norm_w = dev(mn);
        L.in_proj_w = dev(ip);
        L.out_proj_w = dev(op);
        if (wdt == LSSM_DTYPE_INT4_B32 || wdt == LSSM_DTYPE_Q4_G64 || wdt == LSSM_DTYPE_Q8_G32) {
            // scales follow the packed values of the whole tensor
            const uint64_t per = (wdt == LSSM_DTYPE_Q8_G32) ? 1 : 2;
            L.in_proj_s = static_cast<const uint8_t*>(L.in_proj_w) + proj * c.d_model / per;
            L.out_proj_s = static_cast<const uint8_t*>(L.out_proj_w) + uint64_t(c.d_model) * d_inner / per;
        }
    }
    if (wdt == LSSM_DTYPE_INT4_B32) c.wfmt = LSSM_W_Q4_B32;
    else if (wdt == LSSM_DTYPE_Q4_G64) c.wfmt = LSSM_W_Q4_G64;
    else if (wdt == LSSM_DTYPE_Q8_G32) c.wfmt = LSSM_W_Q8_G32;
    else if (wdt == static_cast<int>(act)) c.wfmt = LSSM_W_DENSE;
    else
        return set_error(LSSM_EINVAL,
                         "Mamba2Model: in_proj dtype %d is neither a block format (6, 7, 8) nor the "
                         "activation dtype %u", wdt, act);
    *cfg = c;
    *embed = dev(emb);
    *norm_f = dev(nf);
    *lm_head = dev(head);
    return LSSM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Writer
// ---------------------------------------------------------------------------
struct lssm_ssm_writer {
    int fd = -1;
    std::string path;
    DiskHeader hdr{};
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> by_name;
    bool frozen = false;
    uint64_t file_size = 0;
    int err = LSSM_OK;
    std::string msg;
};

namespace {

int wfail(lssm_ssm_writer* w, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (w->err == LSSM_OK) {
        w->err = code;
        w->msg = buf;
    }
    return set_error(w->err, "%s", w->msg.c_str());
}

bool write_all(int fd, const void* p, uint64_t n, uint64_t off) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    while (n) {
        const ssize_t k = pwrite(fd, b, std::min<uint64_t>(n, uint64_t(1) << 30), static_cast<off_t>(off));
        if (k < 0) {
            if (errno == EINTR) continue;
            return false;
        }
        b += k;
        off += static_cast<uint64_t>(k);
        n -= static_cast<uint64_t>(k);
    }
    return true;
}

// Lay out the index and payloads, write header + index, size the file.
int freeze(lssm_ssm_writer* w) {
    if (w->frozen) return LSSM_OK;
    uint64_t index_bytes = 0;
    for (const Entry& e : w->entries) index_bytes += round_up(sizeof(DiskEntry) + 8ull * e.t.rank + e.name.size(), 8);
    const uint64_t index_off = sizeof(DiskHeader);
    uint64_t off = round_up(index_off + index_bytes, kDataAlign);
    const uint64_t data_off = off;
    for (Entry& e : w->entries) {
        e.t.offset = off;
        off = round_up(off + e.t.nbytes, kDataAlign);
    }
    w->file_size = w->entries.empty() ? data_off
                                      : w->entries.back().t.offset + w->entries.back().t.nbytes;
    DiskHeader& h = w->hdr;
    std::memcpy(h.magic, kMagic, 4);
    h.version = kVersion;
    h.header_size = sizeof(DiskHeader);
    h.n_tensors = static_cast<uint32_t>(w->entries.size());
    h.index_offset = index_off;
    h.data_offset = data_off;
    std::vector<uint8_t> buf(data_off, 0);
    std::memcpy(buf.data(), &h, sizeof(h));
    uint64_t cur = index_off;
    for (const Entry& e : w->entries) {
        DiskEntry d{static_cast<uint32_t>(e.name.size()), e.t.rank, e.t.dtype, 0, e.t.offset, e.t.nbytes};
        std::memcpy(&buf[cur], &d, sizeof(d));
        std::memcpy(&buf[cur + sizeof(d)], e.t.shape, 8ull * e.t.rank);
        std::memcpy(&buf[cur + sizeof(d) + 8ull * e.t.rank], e.name.data(), e.name.size());
        cur += round_up(sizeof(d) + 8ull * e.t.rank + e.name.size(), 8);
    }
    if (ftruncate(w->fd, static_cast<off_t>(w->file_size)) != 0 || !write_all(w->fd, buf.data(), buf.size(), 0))
        return wfail(w, LSSM_EDEVICE, "lssm_ssm_writer: writing '%s' failed: %s", w->path.c_str(), strerror(errno));
    w->frozen = true;
    return LSSM_OK;
}

int put_range(lssm_ssm_writer* w, const Entry& e, uint64_t at, const void* data, uint64_t n) {
    if (at > e.t.nbytes || n > e.t.nbytes - at)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_put: %llu bytes at %llu exceed '%s' (%llu bytes)",
                     (unsigned long long)n, (unsigned long long)at, e.name.c_str(),
                     (unsigned long long)e.t.nbytes);
    if (!write_all(w->fd, data, n, e.t.offset + at))
        return wfail(w, LSSM_EDEVICE, "lssm_ssm_writer: writing '%s' failed: %s", w->path.c_str(), strerror(errno));
    return LSSM_OK;
}

}  // namespace

extern "C" {

int lssm_ssm_writer_create(lssm_ssm_writer** out, const char* path, const lssm_ssm_header* hp) {
    clear_error();
    if (!out || !path || !hp) return set_error(LSSM_EINVAL, "lssm_ssm_writer_create: null argument");
    *out = nullptr;
    auto* w = new lssm_ssm_writer();
    w->path = path;
    w->fd = open(path, O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (w->fd < 0) {
        const int err = errno;
        delete w;
        return set_error(LSSM_EDEVICE, "lssm_ssm_writer_create: open('%s') failed: %s", path, strerror(err));
    }
    DiskHeader& h = w->hdr;
    h.d_model = hp->d_model; h.n_layer = hp->n_layer; h.d_state = hp->d_state; h.d_conv = hp->d_conv;
    h.expand = hp->expand; h.vocab_size = hp->vocab_size; h.n_heads = hp->n_heads; h.d_head = hp->d_head;
    h.chunk_size = hp->chunk_size; h.default_dtype = hp->default_dtype; h.n_groups = hp->n_groups;
    h.norm_before_gate = hp->norm_before_gate;
    *out = w;
    return LSSM_OK;
}

int lssm_ssm_writer_declare(lssm_ssm_writer* w, const char* name, uint32_t dtype, uint32_t rank,
                            const uint64_t* shape) {
    clear_error();
    if (!w) return set_error(LSSM_EINVAL, "lssm_ssm_writer_declare: null writer");
    if (w->err) return set_error(w->err, "%s", w->msg.c_str());
    if (!name || !shape) return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare: null argument");
    if (w->frozen) return wfail(w, LSSM_ESTATE, "lssm_ssm_writer_declare('%s'): index already written", name);
    if (rank == 0 || rank > kMaxRank)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare('%s'): unsupported rank %u", name, rank);
    Entry e;
    e.name = name;
    e.t.dtype = dtype;
    e.t.rank = rank;
    std::memcpy(e.t.shape, shape, 8ull * rank);
    uint64_t n = 0;
    if (!shape_numel(shape, rank, &n)) return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare('%s'): shape overflows", name);
    e.t.nbytes = packed_nbytes(dtype, n);
    if (e.t.nbytes == 0 && n != 0)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare('%s'): unknown dtype %u", name, dtype);
    if ((dtype == LSSM_DTYPE_INT4_B32 || dtype == LSSM_DTYPE_Q8_G32) && n % 32 != 0)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare('%s'): %llu elements is not a multiple of 32", name, (unsigned long long)n);
    if (dtype == LSSM_DTYPE_Q4_G64 && n % 64 != 0)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare('%s'): %llu elements is not a multiple of 64", name, (unsigned long long)n);
    if (!w->by_name.emplace(e.name, w->entries.size()).second)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_declare: duplicate tensor name '%s'", name);
    w->entries.push_back(std::move(e));
    return LSSM_OK;
}

int lssm_ssm_writer_put(lssm_ssm_writer* w, const char* name, const void* data, uint64_t nbytes) {
    clear_error();
    if (!w) return set_error(LSSM_EINVAL, "lssm_ssm_writer_put: null writer");
    if (w->err) return set_error(w->err, "%s", w->msg.c_str());
    if (!name || (!data && nbytes)) return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_put: null argument");
    auto it = w->by_name.find(name);
    if (it == w->by_name.end()) return wfail(w, LSSM_ENOTFOUND, "lssm_ssm_writer_put: '%s' was not declared", name);
    const Entry& e = w->entries[it->second];
    if (nbytes != e.t.nbytes)
        return wfail(w, LSSM_EINVAL, "lssm_ssm_writer_put('%s'): %llu bytes, declared size %llu", name,
                     (unsigned long long)nbytes, (unsigned long long)e.t.nbytes);
    if (int rc = freeze(w)) return rc;
    return put_range(w, e, 0, data, nbytes);
}

int lssm_ssm_writer_finish(lssm_ssm_writer* w) {
    clear_error();
    if (!w) return set_error(LSSM_EINVAL, "lssm_ssm_writer_finish: null writer");
    if (w->err == LSSM_OK) freeze(w);
    if (w->err == LSSM_OK && fsync(w->fd) != 0 && errno != EINVAL)
        wfail(w, LSSM_EDEVICE, "lssm_ssm_writer: fsync('%s') failed: %s", w->path.c_str(), strerror(errno));
    if (w->fd >= 0 && close(w->fd) != 0 && w->err == LSSM_OK)
        wfail(w, LSSM_EDEVICE, "lssm_ssm_writer: close('%s') failed: %s", w->path.c_str(), strerror(errno));
    const int rc = w->err;
    const std::string msg = w->msg;
    if (rc != LSSM_OK) unlink(w->path.c_str());
    delete w;
    if (rc != LSSM_OK) return set_error(rc, "%s", msg.c_str());
    return LSSM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Quantizer and random-init model writer
// ---------------------------------------------------------------------------
namespace {

// fp32 -> fp16 / bf16, round to nearest even.
inline uint16_t f2h(float v) {
    const _Float16 h = static_cast<_Float16>(v);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
inline float h2f(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return static_cast<float>(h);
}
inline uint16_t f2b(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);   // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

void quantize_rows(const float* w, uint64_t N, uint32_t K, uint32_t wfmt, uint8_t* packed,
                   uint16_t* scales) {
    const uint32_t G = wfmt == LSSM_W_Q4_G64 ? 64 : 32;
    const bool q8 = wfmt == LSSM_W_Q8_G32;
    const float qmax = q8 ? 127.0f : 7.0f, qmin = q8 ? -128.0f : -8.0f;
    for (uint64_t n = 0; n < N; ++n) {
        const float* row = w + n * K;
        for (uint32_t g = 0; g < K / G; ++g) {
            float amax = 0.0f;
            for (uint32_t i = 0; i < G; ++i) amax = std::max(amax, std::fabs(row[g * G + i]));
            const float scale = std::max(amax, 1e-12f) / qmax;
            scales[n * (K / G) + g] = f2h(scale);
            for (uint32_t i = 0; i < G; ++i) {
                const uint32_t k = g * G + i;
                const float q = std::min(std::max(std::nearbyint(row[k] / scale), qmin), qmax);
                const int qi = static_cast<int>(q);
                if (q8) {
                    packed[n * K + k] = static_cast<uint8_t>(static_cast<int8_t>(qi));
                } else {
                    uint8_t& byte = packed[(n * K + k) / 2];
                    const uint8_t nib = static_cast<uint8_t>(qi & 0xF);
                    byte = (k & 1) ? static_cast<uint8_t>((byte & 0x0F) | (nib << 4))
                                   : static_cast<uint8_t>((byte & 0xF0) | nib);
                }
            }
        }
    }
}

inline uint64_t mix64(uint64_t x) {   // splitmix64 finaliser
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

inline double unit(std::mt19937_64& g) { return static_cast<double>(g() >> 11) * 0x1.0p-53; }

// out[i] = mean + std * N(0,1) (kind 0) or u ~ U[0,1) (kind 1); blocks of
// 2^16 values, each from its own generator keyed by (key, block), spread over
// threads, so the values do not depend on the thread count.
void fill(float* out, uint64_t n, uint64_t key, int kind, double mean, double stdv) {
    constexpr uint64_t kBlock = uint64_t(1) << 16;
    const uint64_t nb = (n + kBlock - 1) / kBlock;
    const unsigned nt = static_cast<unsigned>(std::max<uint64_t>(
        1, std::min<uint64_t>(nb, std::min(16u, std::max(1u, std::thread::hardware_concurrency())))));
    auto work = [&](unsigned t) {
        for (uint64_t b = t; b < nb; b += nt) {
            std::mt19937_64 g(mix64(key ^ mix64(b)));
            const uint64_t lo = b * kBlock, hi = std::min(n, lo + kBlock);
            for (uint64_t i = lo; i < hi; i += 2) {
                if (kind == 1) {
                    out[i] = static_cast<float>(unit(g));
                    if (i + 1 < hi) out[i + 1] = static_cast<float>(unit(g));
                    continue;
                }
                const double u1 = 1.0 - unit(g), u2 = unit(g);   // u1 in (0, 1]
                const double r = std::sqrt(-2.0 * std::log(u1)), a = 6.283185307179586 * u2;
                out[i] = static_cast<float>(mean + stdv * r * std::cos(a));
                if (i + 1 < hi) out[i + 1] = static_cast<float>(mean + stdv * r * std::sin(a));
            }
        }
    };
    std::vector<std::thread> th;
    for (unsigned t = 1; t < nt; ++t) th.emplace_back(work, t);
    work(0);
    for (auto& x : th) x.join();
}

std::vector<uint8_t> to_act(const float* v, uint64_t n, uint32_t act) {
    std::vector<uint8_t> out(n * (act == LSSM_F32 ? 4 : 2));
    if (act == LSSM_F32) {
        std::memcpy(out.data(), v, n * 4);
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(out.data());
        for (uint64_t i = 0; i < n; ++i) o[i] = act == LSSM_F16 ? f2h(v[i]) : f2b(v[i]);
    }
    return out;
}

}  // namespace

extern "C" {

int lssm_quantize(const float* w, uint32_t N, uint32_t K, uint32_t wfmt, uint8_t* packed,
                  uint16_t* scales) {
    clear_error();
    LSSM_REQUIRE(w && packed && scales, "lssm_quantize: null argument");
    LSSM_REQUIRE(wfmt == LSSM_W_Q4_B32 || wfmt == LSSM_W_Q4_G64 || wfmt == LSSM_W_Q8_G32,
                 "lssm_quantize: wfmt %u is not a block format", wfmt);
    const uint32_t G = wfmt_group(static_cast<int>(wfmt));
    LSSM_REQUIRE(K % G == 0, "lssm_quantize: K=%u not divisible by the group %u", K, G);
    if (wfmt != LSSM_W_Q8_G32) std::memset(packed, 0, uint64_t(N) * K / 2);
    quantize_rows(w, N, K, wfmt, packed, scales);
    return LSSM_OK;
}

int lssm_ssm_write_random(const char* path, const lssm_model_config* cfg, uint64_t seed) {
    clear_error();
    LSSM_REQUIRE(path && cfg, "lssm_ssm_write_random: null argument");
    const lssm_model_config c = *cfg;
    LSSM_REQUIRE(valid_act(static_cast<int>(c.act)), "lssm_ssm_write_random: act %u", c.act);
    LSSM_REQUIRE(valid_wfmt(static_cast<int>(c.wfmt)), "lssm_ssm_write_random: wfmt %u", c.wfmt);
    const uint32_t G = c.n_groups ? c.n_groups : 1;
    const uint64_t d_inner = uint64_t(c.expand) * c.d_model;
    const uint64_t xbc = d_inner + 2ull * G * c.d_state, proj = d_inner + xbc + c.n_heads;
    LSSM_REQUIRE(c.d_model && c.n_layer && c.n_heads && c.vocab_size && c.d_conv &&
                 uint64_t(c.n_heads) * c.d_head == d_inner,
                 "lssm_ssm_write_random: inconsistent shape");
    const uint32_t gq = wfmt_group(static_cast<int>(c.wfmt));
    LSSM_REQUIRE(c.wfmt == LSSM_W_DENSE || (c.d_model % gq == 0 && d_inner % gq == 0),
                 "lssm_ssm_write_random: d_model / d_inner not divisible by the group %u", gq);
    const uint32_t act = c.act;
    const uint32_t wdt = c.wfmt == LSSM_W_DENSE ? act : c.wfmt;   // format codes equal dtype codes

    lssm_ssm_header hp{};
    hp.d_model = c.d_model; hp.n_layer = c.n_layer; hp.d_state = c.d_state; hp.d_conv = c.d_conv;
    hp.expand = c.expand; hp.vocab_size = c.vocab_size; hp.n_heads = c.n_heads; hp.d_head = c.d_head;
    hp.chunk_size = c.chunk_size; hp.default_dtype = act; hp.n_groups = G; hp.norm_before_gate = 0;
    lssm_ssm_writer* w = nullptr;
    if (int rc = lssm_ssm_writer_create(&w, path, &hp)) return rc;

    struct Spec {
        std::string name;
        uint32_t dtype, rank;
        uint64_t shape[4];
    };
    std::vector<Spec> specs;
    specs.push_back({"backbone.embeddings.weight", act, 2, {c.vocab_size, c.d_model}});
    for (uint32_t i = 0; i < c.n_layer; ++i) {   // the exporter's (state-dict) order
        const std::string p = "backbone.layers." + std::to_string(i) + ".";
        specs.push_back({p + "mixer.dt_bias", act, 1, {c.n_heads}});
        specs.push_back({p + "mixer.A_log", act, 1, {c.n_heads}});
        specs.push_back({p + "mixer.D", act, 1, {c.n_heads}});
        specs.push_back({p + "mixer.conv1d.weight", act, 3, {xbc, 1, c.d_conv}});
        specs.push_back({p + "mixer.conv1d.bias", act, 1, {xbc}});
        specs.push_back({p + "mixer.in_proj.weight", wdt, 2, {proj, c.d_model}});
        specs.push_back({p + "mixer.norm.weight", act, 1, {d_inner}});
        specs.push_back({p + "mixer.out_proj.weight", wdt, 2, {c.d_model, d_inner}});
        specs.push_back({p + "norm.weight", act, 1, {c.d_model}});
    }
    specs.push_back({"backbone.norm_f.weight", act, 1, {c.d_model}});
    for (const Spec& s : specs)
        if (lssm_ssm_writer_declare(w, s.name.c_str(), s.dtype, s.rank, s.shape) != LSSM_OK)
            return lssm_ssm_writer_finish(w);

    std::vector<float> buf;
    std::vector<uint8_t> packed;
    for (size_t ti = 0; ti < specs.size(); ++ti) {
        const Spec& s = specs[ti];
        uint64_t n = 1;
        for (uint32_t r = 0; r < s.rank; ++r) n *= s.shape[r];
        buf.resize(n);
        const uint64_t key = mix64(seed) ^ mix64(0x5353u + ti);
        const auto ends = [&](const char* suf) {
            const size_t k = std::strlen(suf);
            return s.name.size() >= k && s.name.compare(s.name.size() - k, k, suf) == 0;
        };
        const bool linear = ends(".in_proj.weight") || ends(".out_proj.weight");
        if (linear) {
            fill(buf.data(), n, key, 0, 0.0, 0.02);
            for (float& v : buf) v = h2f(f2h(v));   // the exporter's input is an fp16 tensor
        } else if (ends(".dt_bias")) {
            fill(buf.data(), n, key, 1, 0.0, 0.0);
            for (float& v : buf) {
                const double dt = std::exp(v * (std::log(0.1) - std::log(1e-3)) + std::log(1e-3));
                v = static_cast<float>(dt + std::log(-std::expm1(-dt)));
            }
        } else if (ends(".A_log")) {
            fill(buf.data(), n, key, 1, 0.0, 0.0);
            for (float& v : buf) v = static_cast<float>(std::log(1.0 + 15.0 * v));
        } else if (ends("norm.weight") || ends("norm_f.weight") || ends(".D")) {
            fill(buf.data(), n, key, 0, 1.0, 0.1);
        } else if (ends(".conv1d.weight")) {
            fill(buf.data(), n, key, 0, 0.0, 0.3);
        } else if (ends(".conv1d.bias")) {
            fill(buf.data(), n, key, 0, 0.0, 0.1);
        } else {   // embeddings
            fill(buf.data(), n, key, 0, 0.0, 0.02);
        }
        int rc;
        if (linear && c.wfmt != LSSM_W_DENSE) {
            const uint64_t N = s.shape[0];
            const uint32_t K = static_cast<uint32_t>(s.shape[1]);
            const uint64_t pb = (c.wfmt == LSSM_W_Q8_G32) ? n : n / 2;
            packed.assign(pb + n / gq * 2, 0);
            quantize_rows(buf.data(), N, K, c.wfmt, packed.data(),
                          reinterpret_cast<uint16_t*>(packed.data() + pb));
            rc = lssm_ssm_writer_put(w, s.name.c_str(), packed.data(), packed.size());
        } else {
            const std::vector<uint8_t> bytes = to_act(buf.data(), n, act);
            rc = lssm_ssm_writer_put(w, s.name.c_str(), bytes.data(), bytes.size());
        }
        if (rc != LSSM_OK) return lssm_ssm_writer_finish(w);
    }
    return lssm_ssm_writer_finish(w);
}

}  // extern "C"
