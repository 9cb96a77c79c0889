// nf4_probe.hpp -- the streaming read / copy probe (measurement only).
#pragma once

#include "nf4_common.hpp"

namespace unifur {

// n16 16-byte units from src: read (dst == null; sink receives a value only
// if the loaded data XOR to `never`) or copied to dst; `grid` workgroups.
hipError_t launch_stream_probe(const void* src, size_t n16, void* dst, uint32_t never, uint32_t* sink, int grid,
                               hipStream_t stream);

}  // namespace unifur
