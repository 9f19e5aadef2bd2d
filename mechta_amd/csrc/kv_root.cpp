// kv_root.cpp -- root files: the reference's on-disk prefix cache (write_root_file / read_root_file,
// session.rs:92-129) for the KV part of the model state (read_root / write_root, engine.rs:782-823).
//
// Byte layout (the reference's, so files are interchangeable):
//   "MECHTA-ROOT-1\n" | u64 p | u64 ns | u64 nk | p x u32 tokens | ns x SSM vector | ns x conv vector |
//   nk x (K vector, V vector),  vector = u64 n | n x 32-bit word,  all little-endian.
// The KV words are positions [0, p) of one attention layer in the position-major order of the reference's buffers
// ([pos][kvh][256], kv.wgsl:7-8): f32 values, or pairs of f16 bits (element 2t in the low half of word t).
// The store keeps its own tiled layout; read_rows / write_rows (kv_append.hip) convert on the device.
#include <hip/hip_runtime.h>

#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "mkv_store.h"

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "root files are little-endian; so is this host");

using namespace mkv;

namespace {

const char HEADER[] = "MECHTA-ROOT-1\n";
constexpr size_t HLEN = sizeof(HEADER) - 1;  // 14

uint64_t kv_words_of(int fmt, int p) { return fmt == 0 ? (uint64_t)p * 256 : (uint64_t)p * 512; }

struct FileCloser {
    FILE* f;
    ~FileCloser() {
        if (f) fclose(f);
    }
};

int write_file(const std::string& path, const char* buf, size_t n, std::string& err) {
    const std::string tmp = path + ".tmp";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) {
        err = "mkv_root_save: cannot create " + tmp;
        return MKV_E_IO;
    }
    size_t done = 0;
    while (done < n) {
        const size_t w = fwrite(buf + done, 1, n - done < (64u << 20) ? n - done : (64u << 20), f);
        if (w == 0) break;
        done += w;
    }
    const bool ok = done == n && fflush(f) == 0;
    if (fclose(f) != 0 || !ok) {
        remove(tmp.c_str());
        err = "mkv_root_save: write failed: " + tmp;
        return MKV_E_IO;
    }
    if (rename(tmp.c_str(), path.c_str()) != 0) {
        remove(tmp.c_str());
        err = "mkv_root_save: cannot rename to " + path;
        return MKV_E_IO;
    }
    return MKV_OK;
}

// The counts of a root file, each checked against the file's size.
struct RootInfo {
    uint64_t p = 0, ns = 0, nk = 0, kv_words = 0;
    std::vector<uint64_t> ssm, conv;
};

int scan(const char* path, RootInfo& ri) {
    FILE* f = fopen(path, "rb");
    if (!f) return fail(MKV_E_IO, "root file %s: cannot open", path);
    FileCloser fc{f};
    if (fseeko(f, 0, SEEK_END) != 0) return fail(MKV_E_IO, "root file %s: cannot seek", path);
    const uint64_t size = (uint64_t)ftello(f);
    rewind(f);
    char h[HLEN];
    if (fread(h, 1, HLEN, f) != HLEN || memcmp(h, HEADER, HLEN) != 0)
        return fail(MKV_E_IO, "root file %s: not a MECHTA-ROOT-1 file", path);
    uint64_t off = HLEN;
    auto get64 = [&](uint64_t& x) {
        if (off + 8 > size || fseeko(f, (off_t)off, SEEK_SET) != 0 || fread(&x, 8, 1, f) != 1) return false;
        off += 8;
        return true;
    };
    auto skip_words = [&](uint64_t n) {
        if (n > (size - off) / 4) return false;
        off += 4 * n;
        return true;
    };
    if (!get64(ri.p) || !get64(ri.ns) || !get64(ri.nk)) return fail(MKV_E_IO, "root file %s: truncated header", path);
    if (ri.p > (1u << 30) || ri.ns > (1u << 20) || ri.nk > (1u << 16) || !skip_words(ri.p))
        return fail(MKV_E_IO, "root file %s: truncated or implausible counts", path);
    ri.ssm.resize(ri.ns);
    ri.conv.resize(ri.ns);
    for (auto* v : {&ri.ssm, &ri.conv})
        for (auto& n : *v)
            if (!get64(n) || !skip_words(n)) return fail(MKV_E_IO, "root file %s: truncated state vector", path);
    for (uint64_t j = 0; j < 2 * ri.nk; j++) {
        uint64_t n;
        if (!get64(n) || !skip_words(n)) return fail(MKV_E_IO, "root file %s: truncated KV vector", path);
        if (j > 0 && n != ri.kv_words) return fail(MKV_E_IO, "root file %s: KV vectors of unequal length", path);
        ri.kv_words = n;
    }
    return MKV_OK;
}

}  // namespace

namespace mkv {
void root_join(mkv_store* h) {
    if (h->root_thread.joinable()) h->root_thread.join();
}

void root_free(mkv_store* h) {
    root_join(h);
    if (h->root_host) (void)hipHostFree(h->root_host);
    h->root_host = nullptr;
    h->root_cap = 0;
}

// The handle's pinned host buffer of at least `bytes` (kept for later calls, grown only when a larger one is needed);
// the caller has joined the background write that may be reading it.
char* root_pinned(mkv_store* h, size_t bytes) {
    if (bytes <= h->root_cap) return (char*)h->root_host;
    if (h->root_host) (void)hipHostFree(h->root_host);
    h->root_host = nullptr;
    h->root_cap = 0;
    if (hipHostMalloc(&h->root_host, bytes, hipHostMallocDefault) != hipSuccess) {
        h->root_host = nullptr;
        (void)hipGetLastError();
        return nullptr;
    }
    h->root_cap = bytes;
    return (char*)h->root_host;
}

// Positions per run of the row conversion staged in the store's prefill workspace (device): the position-major words
// of `run` positions of one plane pair fit it.
int staging_run(const mkv_store* h) {
    const size_t per_pos = (size_t)KVH * HD * h->g.bpe();
    return (int)std::min<size_t>((size_t)h->g.ctx, h->pws_floats * sizeof(float) / per_pos);
}
}  // namespace mkv

uint64_t mkv_root_key(const uint32_t* tokens, size_t n) {
    uint64_t x = 0xcbf29ce484222325ull;  // FNV-1a 64: offset basis, then per byte xor and multiply by the prime
    for (size_t i = 0; i < n; i++)
        for (int b = 0; b < 4; b++) {
            x ^= (tokens[i] >> (8 * b)) & 0xff;
            x *= 0x100000001b3ull;
        }
    return x;
}

int mkv_root_save(mkv_t* h, const char* path, int p, const uint32_t* tokens, int ns, const float* const* ssm,
                  const uint64_t* ssm_words, const float* const* conv, const uint64_t* conv_words, int background) {
    if (!h || !path) return fail(MKV_E_ARG, "mkv_root_save: NULL argument");
    if (p < 0 || p > h->g.ctx) return fail(MKV_E_POS, "mkv_root_save: p = %d", p);
    for (int l = 0; l < h->g.layers; l++)
        if (p > h->len[l]) return fail(MKV_E_POS, "mkv_root_save: p = %d past the written length %d of layer %d", p,
                                       h->len[l], l);
    if ((p > 0 && !tokens) || ns < 0 || (ns > 0 && (!ssm || !ssm_words || !conv || !conv_words)))
        return fail(MKV_E_ARG, "mkv_root_save: NULL tokens or state arrays");
    for (int i = 0; i < ns; i++)
        if ((ssm_words[i] && !ssm[i]) || (conv_words[i] && !conv[i]))
            return fail(MKV_E_ARG, "mkv_root_save: NULL state vector %d", i);
    root_join(h);
    h->root_rc = MKV_OK;

    const int nk = h->g.layers;
    const uint64_t kw = kv_words_of(h->g.fmt, p);
    size_t total = HLEN + 24 + 4 * (size_t)p + (size_t)nk * 2 * (8 + 4 * kw);
    for (int i = 0; i < ns; i++) total += 16 + 4 * (ssm_words[i] + conv_words[i]);
    char* buf = root_pinned(h, total);
    if (!buf) return fail(MKV_E_NOMEM, "mkv_root_save: %zu bytes of pinned host memory", total);
    size_t off = 0;
    auto put = [&](const void* src, size_t n) {
        if (n) memcpy(buf + off, src, n);
        off += n;
    };
    auto put64 = [&](uint64_t x) { put(&x, 8); };
    put(HEADER, HLEN);
    put64((uint64_t)p);
    put64((uint64_t)ns);
    put64((uint64_t)nk);
    put(tokens, 4 * (size_t)p);
    for (int i = 0; i < ns; i++) {
        put64(ssm_words[i]);
        put(ssm[i], 4 * ssm_words[i]);
    }
    for (int i = 0; i < ns; i++) {
        put64(conv_words[i]);
        put(conv[i], 4 * conv_words[i]);
    }
    // K and V words of every layer: converted to position-major on the device, in runs of positions staged in the
    // store's prefill workspace, then copied into the image
    const int run = staging_run(h);
    const size_t per_pos = (size_t)KVH * HD * h->g.bpe();
    float* stage = h->pws;
    hipError_t e = hipSuccess;
    for (int l = 0; l < nk && e == hipSuccess; l++)
        for (int which = 0; which < 2 && e == hipSuccess; which++) {
            put64(kw);
            for (int p0 = 0; p0 < p && e == hipSuccess; p0 += run) {
                const int p1 = std::min(p, p0 + run);
                e = launch_read_rows(h->g, h->base, l, which, p0, p1, stage, Launch{h->stream});
                if (e == hipSuccess)
                    e = hipMemcpyAsync(buf + off + p0 * per_pos, stage, (p1 - p0) * per_pos, hipMemcpyDeviceToHost,
                                       h->stream);
            }
            off += 4 * kw;
        }
    if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) return hip_fail(e, "mkv_root_save");
    const std::string file(path);
    if (background) {
        h->root_thread = std::thread([h, file, buf, total] {
            std::string err;
            h->root_rc = write_file(file, buf, total, err);
            if (h->root_rc != MKV_OK) snprintf(h->root_err, sizeof h->root_err, "%s", err.c_str());
        });
        return MKV_OK;
    }
    std::string err;
    const int rc = write_file(file, buf, total, err);
    return rc == MKV_OK ? MKV_OK : fail(rc, "%s", err.c_str());
}

int mkv_root_wait(mkv_t* h) {
    if (!h) return fail(MKV_E_ARG, "mkv_root_wait: NULL handle");
    root_join(h);
    const int rc = h->root_rc;
    h->root_rc = MKV_OK;
    return rc == MKV_OK ? MKV_OK : fail(rc, "%s", h->root_err);
}

int mkv_root_info(const char* path, int* p, int* ns, int* nk, uint64_t* kv_words, uint64_t* ssm_words,
                  uint64_t* conv_words, int max_ns) {
    if (!path) return fail(MKV_E_ARG, "mkv_root_info: NULL path");
    RootInfo ri;
    if (int rc = scan(path, ri)) return rc;
    if (p) *p = (int)ri.p;
    if (ns) *ns = (int)ri.ns;
    if (nk) *nk = (int)ri.nk;
    if (kv_words) *kv_words = ri.kv_words;
    for (uint64_t i = 0; i < ri.ns && (int64_t)i < max_ns; i++) {
        if (ssm_words) ssm_words[i] = ri.ssm[i];
        if (conv_words) conv_words[i] = ri.conv[i];
    }
    return MKV_OK;
}

int mkv_root_load(mkv_t* h, const char* path, uint32_t* tokens, float* const* ssm, float* const* conv) {
    if (!h || !path) return fail(MKV_E_ARG, "mkv_root_load: NULL argument");
    RootInfo ri;
    if (int rc = scan(path, ri)) return rc;
    const int p = (int)ri.p;
    if ((int)ri.nk != h->g.layers || p > h->g.ctx || (ri.nk && ri.kv_words != kv_words_of(h->g.fmt, p)))
        return fail(MKV_E_FMT,
                    "mkv_root_load: %s holds %llu layers of %llu words at p = %d; the store has %d layers, ctx %d, "
                    "%llu words per vector at that p",
                    path, (unsigned long long)ri.nk, (unsigned long long)ri.kv_words, p, h->g.layers, h->g.ctx,
                    (unsigned long long)kv_words_of(h->g.fmt, p));
    root_join(h);
    FILE* f = fopen(path, "rb");
    if (!f) return fail(MKV_E_IO, "root file %s: cannot open", path);
    FileCloser fc{f};
    auto read_or_skip = [&](void* dst, uint64_t bytes) {
        if (dst) return fread(dst, 1, bytes, f) == bytes;
        return fseeko(f, (off_t)bytes, SEEK_CUR) == 0;
    };
    bool ok = fseeko(f, (off_t)(HLEN + 24), SEEK_SET) == 0 && read_or_skip(tokens, 4 * ri.p);
    for (uint64_t i = 0; i < ri.ns && ok; i++) ok = read_or_skip(nullptr, 8) && read_or_skip(ssm ? ssm[i] : nullptr, 4 * ri.ssm[i]);
    for (uint64_t i = 0; i < ri.ns && ok; i++)
        ok = read_or_skip(nullptr, 8) && read_or_skip(conv ? conv[i] : nullptr, 4 * ri.conv[i]);
    if (!ok) return fail(MKV_E_IO, "root file %s: read failed", path);
    const uint64_t kw = ri.kv_words;
    if (kw) {
        // one vector at a time, in runs of positions: file -> the handle's pinned buffer -> the prefill workspace
        // (device staging) -> store layout
        const int run = staging_run(h);
        const size_t per_pos = (size_t)KVH * HD * h->g.bpe();
        char* host = root_pinned(h, (size_t)std::min(run, p) * per_pos);
        if (!host) return fail(MKV_E_NOMEM, "mkv_root_load: pinned host memory");
        hipError_t e = hipSuccess;
        for (int l = 0; l < h->g.layers && ok && e == hipSuccess; l++)
            for (int which = 0; which < 2 && ok && e == hipSuccess; which++) {
                ok = read_or_skip(nullptr, 8);
                for (int p0 = 0; p0 < p && ok && e == hipSuccess; p0 += run) {
                    const int p1 = std::min(p, p0 + run);
                    e = hipStreamSynchronize(h->stream);  // the previous run left the pinned buffer
                    ok = e == hipSuccess && read_or_skip(host, (p1 - p0) * per_pos);
                    if (!ok) break;
                    e = hipMemcpyAsync(h->pws, host, (p1 - p0) * per_pos, hipMemcpyHostToDevice, h->stream);
                    if (e == hipSuccess)
                        e = launch_write_rows(h->g, h->base, l, which, p0, p1, h->pws, Launch{h->stream});
                }
            }
        if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
        if (e != hipSuccess) return hip_fail(e, "mkv_root_load");
        if (!ok) return fail(MKV_E_IO, "root file %s: read failed (the store's positions [0, %d) are undefined)", path, p);
    }
    for (int l = 0; l < h->g.layers; l++) h->len[l] = p;
    return MKV_OK;
}

int mkv_root_path(char* out, size_t cap, const char* dir, int fmt, const char* model_path, const uint32_t* tokens,
                  size_t n) {
    if (!out || !dir || !model_path || (!tokens && n > 0)) return fail(MKV_E_ARG, "mkv_root_path: NULL argument");
    if (fmt != MKV_F16 && fmt != MKV_F32) return fail(MKV_E_ARG, "mkv_root_path: format %d", fmt);
    // the model key: every byte of the path is one token (root_key over the bytes widened to u32)
    std::vector<uint32_t> mb;
    for (const unsigned char* c = (const unsigned char*)model_path; *c; c++) mb.push_back(*c);
    char name[64];
    snprintf(name, sizeof name, "root-%s-%016llx-%016llx.bin", fmt == MKV_F16 ? "f16" : "f32",
             (unsigned long long)mkv_root_key(mb.data(), mb.size()), (unsigned long long)mkv_root_key(tokens, n));
    const std::string full = std::string(dir) + "/" + name;
    if (full.size() + 1 > cap) return fail(MKV_E_SIZE, "mkv_root_path: %zu bytes needed, %zu given", full.size() + 1, cap);
    memcpy(out, full.c_str(), full.size() + 1);
    return (int)full.size();
}

int mkv_root_prune(const char* dir, int fmt, int keep) {
    if (!dir || (fmt != MKV_F16 && fmt != MKV_F32)) return fail(MKV_E_ARG, "mkv_root_prune: bad argument");
    keep = std::max(keep, 1);
    const std::string prefix = std::string("root-") + (fmt == MKV_F16 ? "f16" : "f32") + "-";
    DIR* d = opendir(dir);
    if (!d) return 0;
    struct Entry {
        struct timespec mtime;
        std::string path;
    };
    std::vector<Entry> v;
    while (struct dirent* e = readdir(d)) {
        const std::string name = e->d_name;
        if (name.size() < prefix.size() + 4 || name.compare(0, prefix.size(), prefix) != 0 ||
            name.compare(name.size() - 4, 4, ".bin") != 0)
            continue;
        const std::string path = std::string(dir) + "/" + name;
        struct stat st;
        if (stat(path.c_str(), &st) == 0) v.push_back({st.st_mtim, path});
    }
    closedir(d);
    // newest first (the reference sorts by modification time, descending, and skips the first `keep`)
    std::sort(v.begin(), v.end(), [](const Entry& a, const Entry& b) {
        return a.mtime.tv_sec != b.mtime.tv_sec ? a.mtime.tv_sec > b.mtime.tv_sec : a.mtime.tv_nsec > b.mtime.tv_nsec;
    });
    int removed = 0;
    for (size_t i = (size_t)keep; i < v.size(); i++)
        if (unlink(v[i].path.c_str()) == 0) removed++;
    return removed;
}

int mkv_root_touch(const char* path) {
    if (!path) return fail(MKV_E_ARG, "mkv_root_touch: NULL path");
    const int fd = open(path, O_WRONLY | O_APPEND);
    if (fd < 0) return fail(MKV_E_IO, "mkv_root_touch: cannot open %s", path);
    const int rc = futimens(fd, nullptr);  // both times to now
    close(fd);
    return rc == 0 ? MKV_OK : fail(MKV_E_IO, "mkv_root_touch: cannot set the time of %s", path);
}
