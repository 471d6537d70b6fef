/* engine_internal.h - declarations shared by the host engine's translation units. */
#ifndef PRISM_ENGINE_INTERNAL_H
#define PRISM_ENGINE_INTERNAL_H

#include <cstdint>
#include <string>
#include <vector>

#include "prism.h"

namespace prism {

bool shape_supported(const prism_model_desc* d, std::string* why);
int64_t layout_blocks(const prism_model_desc* d, prism_block_offsets* offs);
int validate_blocks(const prism_model_desc* d, const prism_block_offsets* offs, int64_t total,
                    std::string* why);
int validate_adapters(const prism_model_desc* d, const prism_adapter_offsets* a, int64_t total,
                      std::string* why);
int validate_codec(const prism_model_desc* d, const prism_codec_offsets* c, int64_t total, std::string* why);
/* r0 (render) .. r3 (the token grid) of a render size; false (why) if r3 is
 * not the model's grid */
bool codec_resolutions(const prism_model_desc* d, int render_w, int render_h, int* rw, int* rh, std::string* why);
void pack_fragments(const uint16_t* W, int rows, int K, int rows_padded, uint16_t* dst);
/* The LayerNorm affine moved into the weights that consume its output:
 * Wf[o][i] = r16(W[o][i] * gamma[i]), bias_f[o] = bias[o] + sum_i W[o][i] * beta[i]
 * (W row-major [rows][K], fp16; bias fp16). False (why) if a scaled weight
 * overflows fp16. */
bool fold_layernorm(const uint16_t* W, int rows, int K, const uint16_t* gamma, const uint16_t* beta,
                    const uint16_t* bias, uint16_t* Wf, float* bias_f, std::string* why);
float half_to_float(uint16_t h);
uint16_t float_to_half(float f);

/* model sidecar (model_file.cpp) */
int read_model_json(const std::string& text, prism_model_desc* desc, std::vector<prism_block_offsets>* offs,
                    prism_adapter_offsets* ad, bool* has_adapters, int64_t* total, std::string* why);
bool read_text_file(const char* path, std::string* out);
std::string sidecar_path(const char* weights_path);

/* thread-local message for calls that have no context (create, host helpers) */
void set_global_error(const std::string& msg);

}  // namespace prism

#endif
