// gguf_asan_main.cpp -- drives the GGUF reader (inferno.jl_amd/csrc/gguf.hip,
// compiled as plain C++ with AddressSanitizer and UndefinedBehaviorSanitizer
// by tests/test_gguf_asan.py) over every file named on the command line: open,
// header info, every tensor's info, its bytes into an exact and a short buffer,
// the upload hooks (one tensor, then groups of them), close.  Accepting or refusing a file are both fine; an
// out-of-bounds read, a leak-free use after free or undefined behaviour makes
// the sanitizers end the process with a report.  CPU only.
#include "inferno_hip.h"

#include <cstdio>
#include <string>
#include <vector>

static std::string g_err;

// The two hooks gguf.hip takes from api.hip: the error message, and the
// registry upload (no device here).
int ihip_fail_msg(int code, const char *msg)
{
    g_err = msg;
    return code;
}
int ihip_register_device_copy(const void *host, size_t bytes, int, int, int, uint64_t *handle)
{
    // touch every byte the reader hands over, so a range past the mapping is caught
    const unsigned char *p = (const unsigned char *)host;
    unsigned acc = 0;
    for (size_t i = 0; i < bytes; ++i)
        acc += p[i];
    *handle = acc | 1u;
    return IHIP_ERR_NO_DEVICE;
}

int ihip_register_device_group(const void *const *hosts, const size_t *bytes, const int *, int n,
                               int, int, uint64_t *handle)
{
    unsigned acc = 0;
    for (int m = 0; m < n; ++m) {
        const unsigned char *p = (const unsigned char *)hosts[m];
        for (size_t i = 0; i < bytes[m]; ++i)
            acc += p[i];
    }
    *handle = acc | 1u;
    return IHIP_ERR_NO_DEVICE;
}

int main(int argc, char **argv)
{
    if (argc == 2 && std::string(argv[1]) == "--self-check") {
        // one byte past a heap buffer: a live AddressSanitizer must report it
        std::vector<unsigned char> v(16, 1);
        volatile unsigned char *p = v.data();
        std::printf("%d\n", (int)p[16]);
        return 0;
    }
    int accepted = 0, refused = 0;
    for (int a = 1; a < argc; ++a) {
        uint64_t fh = 0;
        if (ihip_gguf_open(argv[a], &fh) != IHIP_OK) {
            ++refused;
            std::printf("%s: refused: %s\n", argv[a], g_err.c_str());
            continue;
        }
        uint32_t version = 0;
        uint64_t alignment = 0, data_offset = 0;
        int64_t count = 0;
        ihip_gguf_info(fh, &version, &alignment, &data_offset, &count);
        for (int64_t i = 0; i < count; ++i) {
            char name[512];
            int type = 0, ndim = 0;
            int64_t dims[4];
            uint64_t offset = 0, nbytes = 0;
            if (ihip_gguf_tensor_info(fh, i, name, sizeof name, &type, &ndim, dims, &offset, &nbytes) != IHIP_OK)
                continue;
            char tiny[4];
            ihip_gguf_tensor_info(fh, i, tiny, sizeof tiny, &type, &ndim, dims, &offset, &nbytes);
            std::vector<unsigned char> buf(nbytes ? nbytes : 1);
            ihip_gguf_tensor_bytes(fh, name, buf.data(), nbytes);
            if (nbytes > 1)
                ihip_gguf_tensor_bytes(fh, name, buf.data(), nbytes - 1);
            uint64_t wh = 0;
            ihip_gguf_upload(fh, name, &wh);
        }
        // group uploads: every tensor at once, then each neighbouring pair
        std::vector<std::string> names;
        for (int64_t i = 0; i < count; ++i) {
            char name[512];
            int type = 0, ndim = 0;
            int64_t dims[4];
            uint64_t offset = 0, nbytes = 0;
            if (ihip_gguf_tensor_info(fh, i, name, sizeof name, &type, &ndim, dims, &offset, &nbytes) == IHIP_OK)
                names.push_back(name);
        }
        std::vector<const char *> np;
        for (const std::string &n : names)
            np.push_back(n.c_str());
        uint64_t gh = 0;
        if (!np.empty())
            ihip_gguf_upload_group(fh, np.data(), (int)np.size(), &gh);
        for (size_t i = 0; i + 1 < np.size(); ++i)
            ihip_gguf_upload_group(fh, np.data() + i, 2, &gh);
        ihip_gguf_tensor_info(fh, count, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr);
        ihip_gguf_close(fh);
        ++accepted;
        std::printf("%s: accepted v%u, %lld tensors\n", argv[a], version, (long long)count);
    }
    std::printf("accepted %d refused %d\n", accepted, refused);
    return 0;
}
