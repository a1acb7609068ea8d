// gguf.hip -- GGUF file reader feeding the device weight registry (host code).
//
// Follows src/GGUF.jl:119-165 (read_gguf) and src/LoaderCPU.jl:125-163 of
// Inferno.jl: magic "GGUF", version, tensor and key/value counts, the
// key/value section (only general.alignment is kept), the tensor infos
// (name, dims with dims[0] = ne0 = inner, GGML type, offset relative to the
// data section), then the data section at the next multiple of
// general.alignment (default 32).  The file is memory-mapped read-only.
//
// Differences from the reference, all in the direction of refusing bad input:
// every read is bounds-checked against the file size; a tensor's byte size is
// its block count times the block size of its type (src/GGUF.jl:186-205
// returns elements * 4 bytes for every type, which over-reads quantized
// tensors); a tensor whose bytes run past the end of the file is an error;
// versions other than 2 and 3 are refused (version 1 has 32-bit counts, which
// the reference would misread after a warning).
#include "inferno_hip.h"

#include <cstdint>
#include <cstring>
#include <fcntl.h>
#include <mutex>
#include <string>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <unordered_map>
#include <vector>

namespace ihip_gguf {

struct Tensor {
    std::string name;
    int ndim = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    int type = 0;
    uint64_t offset = 0; // relative to the data section
    uint64_t nbytes = 0; // 0: a type whose block size is not known here
};

struct File {
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
};

// Block geometry of the GGML types (src/GGUF.jl:25-60): elements, bytes.
bool type_geometry(int t, int64_t &elems, int64_t &bytes)
{
    switch (t) {
    case 0: elems = 1; bytes = 4; return true;     // F32
    case 1: elems = 1; bytes = 2; return true;     // F16
    case 8: elems = 32; bytes = 34; return true;   // Q8_0
    case 12: elems = 256; bytes = 144; return true; // Q4_K
    case 13: elems = 256; bytes = 176; return true; // Q5_K
    case 14: elems = 256; bytes = 210; return true; // Q6_K
    case 20: elems = 32; bytes = 18; return true;  // IQ4_NL
    case 24: elems = 1; bytes = 1; return true;    // I8
    case 25: elems = 1; bytes = 2; return true;    // I16
    case 26: elems = 1; bytes = 4; return true;    // I32
    case 27: elems = 1; bytes = 8; return true;    // I64
    case 28: elems = 1; bytes = 8; return true;    // F64
    case 30: elems = 1; bytes = 2; return true;    // BF16
    default: return false;
    }
}

class Reader {
  public:
    Reader(const uint8_t *p, size_t n) : p_(p), n_(n) {}
    bool ok() const { return ok_; }
    size_t pos() const { return pos_; }
    const char *why() const { return why_; }

    template <typename T>
    T get()
    {
        T v{};
        if (!need(sizeof(T)))
            return v;
        memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    bool skip(uint64_t k)
    {
        if (!need(k))
            return false;
        pos_ += (size_t)k;
        return true;
    }
    // src/GGUF.jl:74-80: length-prefixed, at most 1 MiB
    bool string(std::string *out)
    {
        const uint64_t len = get<uint64_t>();
        if (!ok_)
            return false;
        if (len > 1048576)
            return fail("string longer than 1 MiB");
        if (!need(len))
            return false;
        if (out)
            out->assign(reinterpret_cast<const char *>(p_ + pos_), (size_t)len);
        pos_ += (size_t)len;
        return true;
    }
    // src/GGUF.jl:82-116; the value of an integer-typed key is returned in
    // *ival when the caller asks for it
    bool value(uint32_t type, int depth, bool *is_int, uint64_t *ival)
    {
        if (depth > 8)
            return fail("arrays nested too deeply");
        if (is_int)
            *is_int = false;
        switch (type) {
        case 0: return scalar<uint8_t>(is_int, ival);
        case 1: return scalar<int8_t>(is_int, ival);
        case 2: return scalar<uint16_t>(is_int, ival);
        case 3: return scalar<int16_t>(is_int, ival);
        case 4: return scalar<uint32_t>(is_int, ival);
        case 5: return scalar<int32_t>(is_int, ival);
        case 6: return skip(4); // float32
        case 7: return skip(1); // bool
        case 8: return string(nullptr);
        case 9: {
            const uint32_t at = get<uint32_t>();
            const uint64_t len = get<uint64_t>();
            if (!ok_)
                return false;
            for (uint64_t i = 0; i < len; ++i)
                if (!value(at, depth + 1, nullptr, nullptr))
                    return false;
            return true;
        }
        case 10: return scalar<uint64_t>(is_int, ival);
        case 11: return scalar<int64_t>(is_int, ival);
        case 12: return skip(8); // float64
        default: return fail("unknown GGUF value type");
        }
    }
    bool fail(const char *why)
    {
        if (ok_)
            why_ = why;
        ok_ = false;
        return false;
    }

  private:
    template <typename T>
    bool scalar(bool *is_int, uint64_t *ival)
    {
        const T v = get<T>();
        if (!ok_)
            return false;
        if (is_int) {
            *is_int = true;
            *ival = (uint64_t)(int64_t)v;
        }
        return true;
    }
    bool need(uint64_t k)
    {
        if (!ok_)
            return false;
        if (k > n_ - pos_)
            return fail("file ends inside the header");
        return true;
    }
    const uint8_t *p_;
    size_t n_, pos_ = 0;
    bool ok_ = true;
    const char *why_ = "";
};

std::mutex g_mu;
std::unordered_map<uint64_t, File> g_files;
uint64_t g_next = 1;

int parse(File &f, std::string &err)
{
    Reader r(f.map, f.size);
    if (r.get<uint32_t>() != 0x46554747u || !r.ok()) {
        err = "not a GGUF file (bad magic)";
        return IHIP_ERR_INVALID;
    }
    f.version = r.get<uint32_t>();
    if (r.ok() && f.version != 2 && f.version != 3) {
        err = "unsupported GGUF version " + std::to_string(f.version);
        return IHIP_ERR_INVALID;
    }
    const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    for (uint64_t i = 0; r.ok() && i < nkv; ++i) {
        std::string key;
        r.string(&key);
        const uint32_t vt = r.get<uint32_t>();
        bool is_int = false;
        uint64_t iv = 0;
        r.value(vt, 0, &is_int, &iv);
        if (r.ok() && key == "general.alignment") {
            if (!is_int || iv == 0 || iv > (1u << 20)) {
                err = "general.alignment must be a positive integer";
                return IHIP_ERR_INVALID;
            }
            f.alignment = iv;
        }
    }
    if (r.ok() && nt > (f.size / 24)) // a tensor info takes at least 24 bytes
        r.fail("tensor count larger than the file can hold");
    for (uint64_t i = 0; r.ok() && i < nt; ++i) {
        Tensor t;
        r.string(&t.name);
        const uint32_t nd = r.get<uint32_t>();
        if (r.ok() && (nd == 0 || nd > 4))
            r.fail("tensor rank must be 1..4");
        for (uint32_t d = 0; r.ok() && d < nd; ++d) {
            const uint64_t v = r.get<uint64_t>();
            if (v == 0 || v > (1ull << 40))
                r.fail("tensor dimension out of range");
            t.dims[d] = (int64_t)v;
        }
        t.ndim = (int)nd;
        t.type = (int)r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok())
            break;
        int64_t be = 0, bb = 0;
        if (type_geometry(t.type, be, bb)) {
            const int64_t n = t.dims[0] * t.dims[1] * t.dims[2] * t.dims[3];
            if (t.dims[0] % be) {
                err = "tensor " + t.name + ": ne0 is not a multiple of the block size";
                return IHIP_ERR_INVALID;
            }
            t.nbytes = (uint64_t)(n / be) * (uint64_t)bb;
        }
        if (f.by_name.count(t.name)) {
            err = "duplicate tensor name " + t.name;
            return IHIP_ERR_INVALID;
        }
        f.by_name[t.name] = f.tensors.size();
        f.tensors.push_back(t);
    }
    if (!r.ok()) {
        err = r.why();
        return IHIP_ERR_INVALID;
    }
    // src/GGUF.jl:153-157: the data section starts at the next multiple of
    // the alignment
    const uint64_t pos = r.pos();
    f.data_offset = (pos + f.alignment - 1) / f.alignment * f.alignment;
    if (f.data_offset > f.size) {
        err = "file ends before its data section";
        return IHIP_ERR_INVALID;
    }
    for (const Tensor &t : f.tensors) {
        const uint64_t avail = f.size - f.data_offset;
        if (t.offset > avail || t.nbytes > avail - t.offset) {
            err = "tensor " + t.name + " runs past the end of the file";
            return IHIP_ERR_INVALID;
        }
    }
    return IHIP_OK;
}

} // namespace ihip_gguf

// Internal hooks of api.hip: error reporting and registry upload.
int ihip_fail_msg(int code, const char *msg);
int ihip_register_device_copy(const void *host, size_t bytes, int type, int inner, int outer,
                              uint64_t *handle);
int ihip_register_device_group(const void *const *hosts, const size_t *bytes, const int *outers,
                               int n, int type, int inner, uint64_t *handle);

using namespace ihip_gguf;

extern "C" {

int ihip_gguf_open(const char *path, uint64_t *file_handle)
{
    if (!path || !file_handle)
        return ihip_fail_msg(IHIP_ERR_INVALID, "null pointer");
    const int fd = open(path, O_RDONLY);
    if (fd < 0)
        return ihip_fail_msg(IHIP_ERR_INVALID, (std::string("cannot open ") + path).c_str());
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return ihip_fail_msg(IHIP_ERR_INVALID, "not a GGUF file (too short)");
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED)
        return ihip_fail_msg(IHIP_ERR_INVALID, "mmap failed");
    File f;
    f.map = static_cast<const uint8_t *>(m);
    f.size = (size_t)st.st_size;
    std::string err;
    const int rc = parse(f, err);
    if (rc != IHIP_OK) {
        munmap(m, f.size);
        return ihip_fail_msg(rc, err.c_str());
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const uint64_t h = g_next++;
    g_files[h] = std::move(f);
    *file_handle = h;
    return IHIP_OK;
}

int ihip_gguf_close(uint64_t file_handle)
{
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_files.find(file_handle);
    if (it == g_files.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, "unknown GGUF handle");
    munmap(const_cast<uint8_t *>(it->second.map), it->second.size);
    g_files.erase(it);
    return IHIP_OK;
}

int ihip_gguf_info(uint64_t file_handle, uint32_t *version, uint64_t *alignment,
                   uint64_t *data_offset, int64_t *tensor_count)
{
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_files.find(file_handle);
    if (it == g_files.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, "unknown GGUF handle");
    const File &f = it->second;
    if (version) *version = f.version;
    if (alignment) *alignment = f.alignment;
    if (data_offset) *data_offset = f.data_offset;
    if (tensor_count) *tensor_count = (int64_t)f.tensors.size();
    return IHIP_OK;
}

int ihip_gguf_tensor_info(uint64_t file_handle, int64_t index, char *name, size_t name_cap,
                          int *ggml_type, int *ndim, int64_t dims[4], uint64_t *offset,
                          uint64_t *nbytes)
{
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_files.find(file_handle);
    if (it == g_files.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, "unknown GGUF handle");
    const File &f = it->second;
    if (index < 0 || index >= (int64_t)f.tensors.size())
        return ihip_fail_msg(IHIP_ERR_INVALID, "tensor index out of range");
    const Tensor &t = f.tensors[(size_t)index];
    if (name) {
        if (name_cap <= t.name.size())
            return ihip_fail_msg(IHIP_ERR_INVALID, "name buffer too small");
        memcpy(name, t.name.c_str(), t.name.size() + 1);
    }
    if (ggml_type) *ggml_type = t.type;
    if (ndim) *ndim = t.ndim;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return IHIP_OK;
}

int ihip_gguf_tensor_bytes(uint64_t file_handle, const char *name, void *dst, size_t dst_bytes)
{
    if (!name || !dst)
        return ihip_fail_msg(IHIP_ERR_INVALID, "null pointer");
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_files.find(file_handle);
    if (it == g_files.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, "unknown GGUF handle");
    const File &f = it->second;
    auto ti = f.by_name.find(name);
    if (ti == f.by_name.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, (std::string("tensor not found: ") + name).c_str());
    const Tensor &t = f.tensors[ti->second];
    if (t.nbytes == 0)
        return ihip_fail_msg(IHIP_ERR_INVALID, "tensor type has no known block size");
    if (dst_bytes < t.nbytes)
        return ihip_fail_msg(IHIP_ERR_INVALID, "destination too small");
    memcpy(dst, f.map + f.data_offset + t.offset, (size_t)t.nbytes);
    return IHIP_OK;
}

int ihip_gguf_upload(uint64_t file_handle, const char *name, uint64_t *weight_handle)
{
    if (!name || !weight_handle)
        return ihip_fail_msg(IHIP_ERR_INVALID, "null pointer");
    // the file stays mapped while the lock is held (a concurrent close waits)
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_files.find(file_handle);
    if (it == g_files.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, "unknown GGUF handle");
    const File &f = it->second;
    auto ti = f.by_name.find(name);
    if (ti == f.by_name.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, (std::string("tensor not found: ") + name).c_str());
    const Tensor &t = f.tensors[ti->second];
    if (t.type != 8 && t.type != 12 && t.type != 13 && t.type != 14 && t.type != 20)
        return ihip_fail_msg(IHIP_ERR_INVALID, "only Q4_K, Q5_K, Q6_K, Q8_0 and IQ4_NL tensors are "
                                               "kept quantized on the device");
    if (t.ndim > 2 || t.dims[0] > INT32_MAX || t.dims[1] > INT32_MAX)
        return ihip_fail_msg(IHIP_ERR_INVALID, "a weight tensor has rank 1 or 2 and int-sized dims");
    // src/LoaderCPU.jl:130-132: inner = ne0, outer = ne1
    return ihip_register_device_copy(f.map + f.data_offset + t.offset, (size_t)t.nbytes, t.type,
                                     (int)t.dims[0], (int)t.dims[1], weight_handle);
}

int ihip_gguf_upload_group(uint64_t file_handle, const char *const *names, int n,
                           uint64_t *weight_handle)
{
    if (!names || !weight_handle)
        return ihip_fail_msg(IHIP_ERR_INVALID, "null pointer");
    if (n <= 0 || n > 64)
        return ihip_fail_msg(IHIP_ERR_INVALID, "a group holds 1 to 64 tensors");
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_files.find(file_handle);
    if (it == g_files.end())
        return ihip_fail_msg(IHIP_ERR_INVALID, "unknown GGUF handle");
    const File &f = it->second;
    std::vector<const void *> hosts((size_t)n);
    std::vector<size_t> bytes((size_t)n);
    std::vector<int> outers((size_t)n);
    int type = -1;
    int64_t inner = -1;
    for (int i = 0; i < n; ++i) {
        if (!names[i])
            return ihip_fail_msg(IHIP_ERR_INVALID, "null tensor name");
        auto ti = f.by_name.find(names[i]);
        if (ti == f.by_name.end())
            return ihip_fail_msg(IHIP_ERR_INVALID, (std::string("tensor not found: ") + names[i]).c_str());
        const Tensor &t = f.tensors[ti->second];
        if (t.type != 8 && t.type != 12 && t.type != 13 && t.type != 14 && t.type != 20)
            return ihip_fail_msg(IHIP_ERR_INVALID, "only Q4_K, Q5_K, Q6_K, Q8_0 and IQ4_NL tensors are "
                                                   "kept quantized on the device");
        if (t.ndim > 2 || t.dims[0] > INT32_MAX || t.dims[1] > INT32_MAX)
            return ihip_fail_msg(IHIP_ERR_INVALID, "a weight tensor has rank 1 or 2 and int-sized dims");
        if (i == 0) {
            type = t.type;
            inner = t.dims[0];
        } else if (t.type != type || t.dims[0] != inner) {
            return ihip_fail_msg(IHIP_ERR_INVALID, "the tensors of a group share one type and one row "
                                                   "length (ne0)");
        }
        hosts[(size_t)i] = f.map + f.data_offset + t.offset;
        bytes[(size_t)i] = (size_t)t.nbytes;
        outers[(size_t)i] = (int)t.dims[1];
    }
    return ihip_register_device_group(hosts.data(), bytes.data(), outers.data(), n, type, (int)inner,
                                      weight_handle);
}

} // extern "C"
