// Host-side checkpoint representation shared by the loader and the engine.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/yuf_engine.h"

namespace yuf {

struct ModelShape {
    int vocab = 0, d = 0, layers = 0, heads = 0, head_size = 0, rosa = 0, low_rank = 0;
    bool tie = true;
    float dropout = 0.0f;
    int midi_offset = 260, midi_vocab = 0;
};

struct TensorInfo {
    std::vector<long long> dims;
    long long offset = 0;  // in floats, into Checkpoint::data
    long long count = 0;
    bool bf16 = false;  // stored as bf16 in the file (version 2); data holds it widened
};

struct Checkpoint {
    ModelShape shape;
    std::map<std::string, TensorInfo> tensors;
    std::vector<float> data;
    std::string header_json;  // the file's UTF-8 JSON header, verbatim
    uint32_t version = 0;
    // Host pointer to a tensor, checking its shape when `dims` is non-empty.
    const float *tensor(const std::string &name, const std::vector<long long> &dims, std::string &err) const;
};

int load_checkpoint(const char *path, Checkpoint &ck);
void fill_config(const ModelShape &s, yuf_model_config &c);
const Checkpoint &checkpoint_of(const yuf_ckpt *h);

}  // namespace yuf
