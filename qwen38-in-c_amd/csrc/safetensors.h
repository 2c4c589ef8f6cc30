// safetensors.h -- index of a safetensors checkpoint (one file or a
// directory of shards), the host side of loading weights straight into HBM.
//
// The format: an 8-byte little-endian header length n, n bytes of JSON
// mapping tensor names to {"dtype", "shape", "data_offsets": [begin, end]}
// (offsets relative to the first byte after the header; "__metadata__" is
// skipped), then the tensor bytes.  Validation follows the reference's
// reader (qwen35-c/src/q35_st.c:86-145): 0 < n <= 16 MiB, known dtypes only,
// offsets inside the file, and end - begin == elements * dtype size.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace q35mm {
namespace st {

// dtype codes in the reference's order (qwen35-c/include/q35/q35_st.h:7-14)
enum Dtype : int { kF8E4M3 = 0, kBF16, kF32, kF16, kI64, kUnknown = -1 };

size_t dtype_size(int d);
const char *dtype_name(int d);

// Shard file names the reference accepts in a directory
// (qwen35-c/src/q35_st.c:64-69): contain ".safetensors", not "json".
bool is_shard_name(const char *name);

struct Tensor {
    std::string name;
    int dtype = kUnknown;
    uint32_t ndim = 0;
    uint32_t shape[8] = {};
    uint32_t file = 0;
    uint64_t offset = 0;   // absolute file offset of the first byte
    uint64_t bytes = 0;
};

enum Status : int { kOk = 0, kOpen, kHeader, kDtype, kRange, kIo };
const char *status_str(int s);

struct Archive {
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, uint32_t> index;

    ~Archive();
    // A .safetensors file, or a directory whose shard files are indexed in
    // name order.  On failure returns the status and names the culprit in msg.
    int open(const char *path, std::string &msg);
    const Tensor *find(const char *name) const;
    // bytes [off, off + len) of tensor t into dst; false on a short read
    bool read(const Tensor &t, uint64_t off, uint64_t len, void *dst) const;
    // the same, split over a small pool of reader threads (page-cache reads
    // run at several times one thread's rate)
    bool read_parallel(const Tensor &t, uint64_t off, uint64_t len, void *dst) const;

  private:
    int index_file(const std::string &path, uint32_t file, std::string &msg);
};

}  // namespace st
}  // namespace q35mm
