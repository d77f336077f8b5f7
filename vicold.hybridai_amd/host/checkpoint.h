// checkpoint.h -- Qwen3.5-style checkpoints on disk: safetensors files
// (io/safetensor_loader.cc:50-406), config.json (models/qwen3_config.cc:
// 12-206) and the checkpoint names of the engine's tensors
// (models/qwen3_weights.cc:196-380).  Host code only; no device calls.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "hai_engine.h"

namespace hybridai::mi355x {

enum class StDType { F32, F16, BF16, F8_E4M3, F8_E5M2, I8, I32, I64, U8, BOOL };
size_t st_dtype_size(StDType t);
const char* st_dtype_name(StDType t);

struct StTensor {
    StDType dtype = StDType::F32;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;  // bytes of the shard's data section
    int shard = 0;
    int64_t numel() const;
    uint64_t bytes() const { return end - begin; }
};

// One safetensors file, or a model directory holding model.safetensors or
// the shards named by model.safetensors.index.json (weight_map).  Headers
// are validated as the reference does: a header length inside the file,
// known dtypes, non-negative dims, offsets inside the data section and a
// byte range equal to shape x dtype size.
class SafeTensors {
public:
    // HAI_OK, HAI_ERR_FILE_NOT_FOUND, HAI_ERR_INVALID_MODEL or
    // HAI_ERR_UNSUPPORTED_DTYPE, with a message in *err
    int open(const std::string& path, std::string* err);
    const StTensor* find(const std::string& name) const;
    // the tensor's bytes into dst (t.bytes() of them)
    int read(const StTensor& t, void* dst, std::string* err) const;
    std::vector<std::string> names() const;

private:
    int parse_shard(const std::string& path, int shard, std::map<std::string, StTensor>* out, std::string* err);
    std::vector<std::string> shard_path_;
    std::vector<uint64_t> shard_data_;  // data section offset of each shard
    std::map<std::string, StTensor> tensors_;
};

// <dir>/config.json (text_config fields first, then the root's) into the
// engine's model config, with the reference's defaults (the 27B shape), its
// head_dim and rope rules, its layer schedule checks and its EOS ids.
// max_positions (optional): max_position_embeddings.
int read_model_config(const std::string& dir, hai_model_config* cfg, std::vector<int64_t>* eos, std::string* err,
                      int64_t* max_positions = nullptr);

// HAI_WEIGHTS_FP8_BLOCK128 when the checkpoint stores the QuantizedWeight
// Linears as F8_E4M3 with weight_scale_inv, HAI_WEIGHTS_BF16 when it stores
// them as BF16; a mixture is an error.
int detect_weight_format(const SafeTensors& st, const hai_model_config& cfg, int32_t* format, std::string* err);

// The checkpoint name of engine tensor id = slot * 64 + kind (slot 0 shared,
// 1 MTP shared, 2 + i layer i, 1024 the MTP decoder layer); empty for an id
// that has none.
std::string checkpoint_name(uint32_t id);

// bf16 bits of a float32 value, when it is exactly representable (the
// engine's weights are bf16; an F32 checkpoint tensor loads only if no
// value would change)
bool exact_bf16(float v, uint16_t* bits);

// file helpers shared by the checkpoint readers
bool is_regular_file(const std::string& path);
bool read_whole_file(const std::string& path, std::string* out);
std::string path_join(const std::string& dir, const std::string& name);

}  // namespace hybridai::mi355x
