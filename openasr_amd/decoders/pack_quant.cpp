// pack_quant.cpp -- the pack writer's per-tensor storage policy
// (crates/openasr-core/src/models/pack_quant.rs:161-213): which ggml type a
// matrix of a given role and shape is written as for a requested pack rung.
// Block quantization needs the quantized axis to be a multiple of 32; the
// K-quant rungs need a multiple of 256 and fall back to Q8_0 otherwise; the
// acoustic-encoder and precision-critical roles are floored at Q8_0; the
// text decoder's matrices, the embedding table and the output projection
// take the requested rung.

#include <cstdint>

#include "openasr_models.h"

namespace {

constexpr int kQ8_0 = 8, kQ3_K = 11, kQ4_K = 12;  // enum ggml_type

bool valid_role(int role) { return role >= OA_ROLE_ACOUSTIC_ENCODER_MATRIX && role <= OA_ROLE_NON_QUANTIZABLE; }

bool requires_q8_floor(int role) {  // pack_quant.rs:164-169
    return role == OA_ROLE_ACOUSTIC_ENCODER_MATRIX || role == OA_ROLE_PRECISION_CRITICAL_MATRIX;
}

}  // namespace

extern "C" {

int oa_classify_quant_tensor_role(const uint64_t * dims, int n_dims, int quantization, int role, int axis) {
    if (!valid_role(role) || quantization < OA_PACK_FP16 || quantization > OA_PACK_Q4_K ||
        (axis != OA_AXIS_FIRST && axis != OA_AXIS_LAST))
        return -2;
    if (role == OA_ROLE_NON_QUANTIZABLE) return -1;
    if (n_dims <= 0 || !dims) return -1;  // no quantized axis
    if (quantization == OA_PACK_FP16) return -1;
    const uint64_t ne0 = axis == OA_AXIS_FIRST ? dims[0] : dims[n_dims - 1];
    if (ne0 % 32 != 0) return -1;
    if (ne0 % 256 == 0 && !requires_q8_floor(role)) {
        if (quantization == OA_PACK_Q3_K) return kQ3_K;
        if (quantization == OA_PACK_Q4_K) return kQ4_K;
    }
    return kQ8_0;
}

int oa_quant_target_write_type(const uint64_t * dims, int n_dims, int quantization, int role, int axis) {
    // pack_quant.rs:127-147: K-quants are matrix formats; only rank-2 tensors
    if (n_dims != 2) {
        if (!valid_role(role) || quantization < OA_PACK_FP16 || quantization > OA_PACK_Q4_K ||
            (axis != OA_AXIS_FIRST && axis != OA_AXIS_LAST))
            return -2;
        return -1;
    }
    return oa_classify_quant_tensor_role(dims, n_dims, quantization, role, axis);
}

}  // extern "C"
