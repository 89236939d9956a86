// packet.hpp -- checks and host expansion of a CSR gradient packet
// (eps::CompactGradients).
//
// The rules are the reference's (src/access/compact_gradients.cpp:10-39):
// dimension 1..4096 and at most 2^20 rows; offsets that start at 0, end at the
// reference count and never decrease; one scale per reference; at most 16 MiB
// of payload (capacity_exceeded); distinct rows; references inside the source
// rows; finite source values; finite scales >= 0.  Expansion sums
// value * scale per reference, in order, from +0.0f, and rejects a
// non-finite sum.
#pragma once

#include <cstdint>

#include "eps/types.hpp"

namespace eps::hipbk {

std::uint64_t PacketBytes(const CompactGradients& packet);
// Throws a Fault on the first rule the packet breaks.
void CheckPacket(const CompactGradients& packet);
RowGradients ExpandPacket(const CompactGradients& packet);

}  // namespace eps::hipbk
