// forward_batch_device.h -- the reference-side binding of the batched layer
// and of the device-resident quantized token table: the code a maintainer of
// the reference adds beside src/forward.cc and src/model.cc to use them.  It
// is compiled against the reference's own headers (with this repository's
// include/cuda_*.h ahead of them, as tests/dropin/Makefile builds the
// overlay library) and linked with the reference's library; its test program
// is tests/dropin/test_forward_batch.cc.
#pragma once
#include "include/batch.h"
#include "include/context.h"
#include "include/model.h"
#include "include/quantized_tensor.h"
#include "include/tensor.h"

namespace yan_lamma {

// ForwardBatch (src/forward.cc:473-488) with its token loop replaced, on a
// model whose weights are on the device (UploadModelWeightToCuda): the batch's
// token rows are gathered at once (from the F32 table, or from the blocks
// UploadTokenTableBlocks left on the device), every layer runs once over all
// of them (CudaForwardLayerBatchDevice), and the last row's logits are
// computed as ForwardToken does (ComputeLogitsDevice, src/forward.cc:425-431).
// Returns the logits of the batch's last token, as ForwardBatch does, and
// leaves the context as ForwardBatch leaves it (pos = the last position,
// tokens appended, K/V rows of every token in the device cache).
//   - Same checks and messages as ForwardBatch / ForwardToken: empty batch,
//     tokens/positions mismatch, token or position out of range.
//   - Without device weights, or with positions that do not increase (where
//     writing every K/V row before attention would differ from the token
//     loop), it is ForwardBatch itself.
//   - Host-to-device copies: the token ids when the batch has more than one
//     token (4 T bytes), and the positions once per layer when they are not
//     consecutive.  Device-to-host: the logits, once.
Tensor ForwardBatchDevice(const Model& model, Context& context, const Batch& batch);

// Keeps the token table on the device as Q8_0 / Q4_0 / Q4_1 blocks instead of
// the F32 copy UploadModelWeightToCuda made (src/model.cc:307): the model's
// "embedding_data_" device weight is replaced by these blocks
// (table.shape == {vocab_size, dim}, rows of ceil(dim / 32) blocks as
// TensorToQ80 / Q40 / Q41 write them, e.g. the GGUF token_embd that
// src/gguf_load.cc:370-404 dequantizes at load).  The F32 device copy is
// released.  EmbeddingDevice's rows then come from the blocks, dequantized
// in the gather, equal to the dequantized table's bit for bit.
void UploadTokenTableBlocks(Model& model, const QuanTensor& table);

// The token table's device weight ("embedding_data_", F32 or blocks), or
// null when the model has none on the device.
const CudaloadWeight* DeviceTokenTable(const Model& model);

}  // namespace yan_lamma
