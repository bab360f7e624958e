// model.h -- the part of the reference's model header the op surface needs.
//
// RoPE pairing layouts, same enumerators and order as the reference
// (include/model.h:37-40 of the reference tree).  The rest of that header
// (model containers, weight upload, runtime counters) belongs to the
// forward pass, which stays the reference's.
#pragma once

namespace yan_lamma {
enum RopeType {
    kNormal,  // adjacent pairs (2i, 2i + 1)
    kNeoX     // half-split pairs (i, i + head_dim / 2)
};
}  // namespace yan_lamma
