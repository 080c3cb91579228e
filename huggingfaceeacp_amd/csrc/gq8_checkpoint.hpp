// gq8_checkpoint.hpp -- checkpoint files on the host: safetensors
// (Lib/HuggingFaceEACP/Model/SafeTensors.h:78-183) mapped rather than read,
// every header field checked before a byte is trusted, and Gemma's
// config.json (Model/GemmaConfig.h:41-92).  Host C++ only.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace gq8 {

// Records a failure as the C ABI's last error and returns the status.
int report(int status, const std::string &message);
// SamplingError's rules (Sampling/Sampler.cpp:28-41): GQ8_OK or GQ8_ERR_ARGUMENT.
int check_sampling(const struct gq8_sampling &options);

// The safetensors dtype tags (Model/TensorType.h:12-27), in that order.
enum Dtype {
    kBool, kU8, kI8, kU16, kI16, kF16, kBF16, kU32, kI32, kF32, kU64, kI64, kF64, kDtypeCount
};
int dtype_bytes(int dtype);
const char *dtype_name(int dtype);

struct TensorInfo {
    std::string name;
    int dtype = kF32;
    std::vector<int64_t> shape;
    uint64_t offset = 0; // from the start of the blob
    uint64_t bytes = 0;
    int64_t elements() const;
};

// One safetensors file: 8 bytes of little-endian header length, the JSON
// header, the blob.  The bytes are a read-only mapping of the file (or an
// owned copy); tensors are sorted by name.
class SafeTensorsFile {
public:
    ~SafeTensorsFile();
    // Status GQ8_OK or a negative status with the error recorded.
    static int open(const std::string &path, SafeTensorsFile **out);
    static int from_bytes(const uint8_t *bytes, uint64_t size, SafeTensorsFile **out);

    const std::vector<TensorInfo> &tensors() const { return tensors_; }
    const std::map<std::string, std::string> &metadata() const { return metadata_; }
    int find(const std::string &name) const; // index, or -1
    const uint8_t *blob_bytes(const TensorInfo &t) const { return data_ + blob_ + t.offset; }

    // Elements [first, first + count) of a floating-point tensor widened to
    // fp32 (F16 and BF16 widen exactly); GQ8_ERR_FORMAT for any other dtype.
    int read_floats(const TensorInfo &t, int64_t first, int64_t count, float *out) const;

private:
    SafeTensorsFile() = default;
    int parse_header();

    const uint8_t *data_ = nullptr;
    uint64_t size_ = 0;
    uint64_t blob_ = 0;
    std::vector<uint8_t> owned_;
    void *mapping_ = nullptr;
    std::vector<TensorInfo> tensors_;
    std::map<std::string, std::string> metadata_;
};

// config.json as GemmaConfig::fromJson reads it (GemmaConfig.cpp:140-205):
// every field defaults to google/gemma-2b's value, model_type must be
// "gemma", token ids are a number or the first of a list.
struct GemmaConfigValues {
    int vocab = 256000, width = 2048, intermediate = 16384, layers = 18, heads = 8, kv_heads = 1,
        head_dim = 256, max_positions = 8192;
    double rms_epsilon = 1.0e-6, rope_theta = 10000.0;
    int bos = 2, eos = 1, pad = 0;
    bool tied = true;
};
int parse_gemma_config(const char *text, size_t length, GemmaConfigValues *out);

} // namespace gq8

struct gq8_safetensors;
namespace gq8 {
const SafeTensorsFile *file_of(const gq8_safetensors *handle);
} // namespace gq8
