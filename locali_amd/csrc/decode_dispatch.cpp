// Decode-path dispatch: picks the (bits, dtype) translation unit and the
// lane geometry for a projection.
#include "launch.hpp"

namespace locali {

hipError_t decode_b2_bf16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b2_f16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b4_bf16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b4_f16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b8_bf16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b8_f16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b3_bf16(int, int, int, const DecodeLaunch &, hipStream_t);
hipError_t decode_b3_f16(int, int, int, const DecodeLaunch &, hipStream_t);

// 16-byte chunks per row and group parts per chunk in the geometry the
// kernels compute in (lane_bits: 3-bit rows in the 4-bit geometry).
int chunks_per_row(const QProj &p) {
    return static_cast<int>(static_cast<int64_t>(p.cols) * lane_bits(p.bits) / 128);
}

int group_parts(const QProj &p) {
    const int vpc = 128 / lane_bits(p.bits);
    return p.group >= vpc ? 1 : vpc / p.group;
}

static hipError_t decode_dispatch(int which, const QProj &p, const DecodeLaunch &L,
                                  hipStream_t st) {
    const int gpc = group_parts(p), cpr = chunks_per_row(p);
    switch (p.bits) {
    case 2: return L.bf16 ? decode_b2_bf16(which, gpc, cpr, L, st) : decode_b2_f16(which, gpc, cpr, L, st);
    case 4: return L.bf16 ? decode_b4_bf16(which, gpc, cpr, L, st) : decode_b4_f16(which, gpc, cpr, L, st);
    case 8: return L.bf16 ? decode_b8_bf16(which, gpc, cpr, L, st) : decode_b8_f16(which, gpc, cpr, L, st);
    case 3: return L.bf16 ? decode_b3_bf16(which, gpc, cpr, L, st) : decode_b3_f16(which, gpc, cpr, L, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gateup_decode(const DecodeLaunch &L, hipStream_t st) {
    if (gateup_diag_eligible(L))
        return L.gate.bits == 2 ? decode_diag_b2(L, st) : L.gate.bits == 3 ? decode_diag_b3(L, st) : decode_diag_b4(L, st);
    return decode_dispatch(0, L.gate, L, st);
}

hipError_t launch_down_combine_decode(const DecodeLaunch &L, hipStream_t st) {
    return decode_dispatch(1, L.down, L, st);
}

}  // namespace locali
