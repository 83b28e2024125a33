/*
 * lutmac_model.h -- .lutmac v1 model files onto the device decoder (C ABI).
 *
 * Replaces load_lutmac (src/format.cpp:292-505) + load_model
 * (src/model.cpp:576-701): parses the file's header and JSON metadata,
 * reads each tensor's 256-weight AoS blocks (the layouts of types.hpp),
 * repacks them into the device tile layout (q|k|v and gate|up fused row-wise)
 * and builds an lmx_decoder (lutmac_decode.h) over them.  Tensor names are
 * matched as load_model matches them; a missing lm_head ties it to the
 * embedding, sharing one device weight instead of a copy.
 *
 * Version 2 adds tensor records {"type": "planes", "format", "group",
 * "rotated", "offset", "planes_bytes", "scales_bytes"} holding canonical
 * planes and per-group scales (any group multiple of 128, RRQ-3), as
 * lutmac_amd/lutmac_file.py writes them from lmx_quantize output; ternary,
 * binary and RRQ planes must be FWHT-rotated, the others not, the embedding
 * never.
 *
 * Supported: decoder-only Llama/Qwen-style models (RMSNorm, SiLU) whose
 * linears and embedding are ternary, binary, 2-bit (Int2Block), 3-bit,
 * 4-bit or 8-bit blocks; norms and biases raw fp32.  5/6-bit tensors, raw
 * fp32 linears or embeddings, GELU/Gemma models return
 * LMX_ERR_UNSUPPORTED_FORMAT.  RoPE is the reference's form (pos / factor,
 * factor = rope_scaling_factor).
 */
#ifndef LUTMAC_MODEL_H
#define LUTMAC_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "lutmac_decode.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lmx_model lmx_model;

/* Loads `path` onto the current device.  max_seq: KV-cache capacity (0 =
 * 2048, the capacity the reference's load_model gives its cache: it never
 * reads the file's max_position_embeddings back, types.hpp:558). */
int lmx_model_load(const char *path, size_t max_seq, lmx_model **out);
int lmx_model_destroy(lmx_model *m);
/* The decoder config derived from the file, and the decoder itself (owned
 * by the model). */
int lmx_model_config(const lmx_model *m, lmx_decoder_config *cfg);
lmx_decoder *lmx_model_decoder(lmx_model *m);
/* Format (lmx_format) of a linear of layer `layer`: which = 0 qkv, 1 o,
 * 2 gate_up, 3 down; layer = -1 for the embedding, -2 for the LM head. */
int lmx_model_weight_format(const lmx_model *m, int layer, int which, int *format);

#ifdef __cplusplus
}
#endif
#endif /* LUTMAC_MODEL_H */
