// Loading a packed model (core.bin, layer_NN.bin, manifest.json of tools/repack.py) into
// HipBackend buffers, and the views the ops need over them.  With 288 GB of HBM the
// whole model stays resident: core.bin in one buffer, each expert layer (128 slots at
// the manifest's stride, 430 MB for Gemma-4 26B) in one buffer, each streamed from disk
// once.
#pragma once
#include <string>

#include "hip_backend.h"
#include "model_info.h"
#include "ops.h"

namespace apex {

// core.bin in one device buffer ("core_weights"); tensors are at their manifest offsets.
inline Buffer *loadCore(HipBackend &backend, const ModelInfo &model) {
    Buffer *b = backend.allocate(model.core_size, "core_weights");
    backend.loadFile(b, 0, model.dir + "/core.bin", 0, model.core_size);
    return b;
}

// layer_NN.bin (all expert slots) in one device buffer ("expert_layers").
inline Buffer *loadExpertLayer(HipBackend &backend, const ModelInfo &model, int layer) {
    const LayerFile &f = model.layers.at(layer);
    Buffer *b = backend.allocate(f.size, "expert_layers");
    backend.loadFile(b, 0, model.dir + "/" + f.file, 0, f.size);
    return b;
}

// The MoE op's view of a loaded expert layer: stride and the six piece offsets
// (tools/repack.py:180-188 piece order).
inline ExpertSlots expertSlots(const ModelInfo &model, Buffer *layer_buffer) {
    auto off = [&](const char *name) { return (uint32_t)model.piece(name).offset; };
    return ExpertSlots{layer_buffer,
                       (uint32_t)model.expert_slot_size,
                       off("gate_proj.weight"),
                       off("gate_proj.scales"),
                       off("up_proj.weight"),
                       off("up_proj.scales"),
                       off("down_proj.weight"),
                       off("down_proj.scales")};
}

// The router tensors of one layer inside the loaded core buffer (tools/out.txt:247-290).
inline RouterWeights routerWeights(const ModelInfo &model, Buffer *core, int layer) {
    const std::string p = "layers." + std::to_string(layer) + ".router.";
    const TensorInfo &w = model.getTensor(p + "proj.weight");
    return RouterWeights{core,
                         model.getTensor(p + "scale").offset,
                         w.offset,
                         model.getTensor(p + "proj.scales").offset,
                         model.getTensor(p + "proj.biases").offset,
                         model.getTensor(p + "per_expert_scale").offset,
                         (uint32_t)w.shape.at(0),
                         (uint32_t)(w.shape.at(1) * 4)};
}

} // namespace apex
