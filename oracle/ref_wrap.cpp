// extern "C" entry points over the reference's own bfp16 packer, compiled from
// its source where it lies (src/npu/bfp16_pack.cpp under the reference tree)
// into oracle/_ref/. Test infrastructure: it produces the golden vectors the
// oracle and the HIP packer are checked against, and nothing else uses it.
#include "bfp16_pack.h"

#include <cstring>
#include <vector>

extern "C" {

void ref_encode_block(const float * x, uint8_t * out) { bfp16_encode_block(x, out); }
void ref_decode_block(const uint8_t * in, float * x) { bfp16_decode_block(in, x); }

void ref_pack_a(const float * x, int64_t M, int64_t K, int m, int k, uint8_t * out) {
    bfp16_tiling t;
    t.m = m;
    t.k = k;
    std::vector<uint8_t> v;
    bfp16_pack_a(x, M, K, t, v, 4);
    std::memcpy(out, v.data(), v.size());
}

void ref_pack_b(const float * w, int64_t N, int64_t K, int n, int k, int cols, uint8_t * out) {
    bfp16_tiling t;
    t.n = n;
    t.k = k;
    t.cols = cols;
    std::vector<uint8_t> v;
    bfp16_pack_b(w, N, K, t, v, 4);
    std::memcpy(out, v.data(), v.size());
}

size_t ref_a_offset(int64_t r, int64_t cb, int64_t K, int m, int k) {
    bfp16_tiling t;
    t.m = m;
    t.k = k;
    return bfp16_a_offset(r, cb, K, t);
}

size_t ref_b_offset(int64_t r, int64_t cb, int64_t N, int64_t K, int n, int k, int cols) {
    bfp16_tiling t;
    t.n = n;
    t.k = k;
    t.cols = cols;
    return bfp16_b_offset(r, cb, N, K, t);
}

void ref_interleave_gate_up(const float * gate, const float * up, int64_t F, int64_t K, float * out) {
    bfp16_interleave_gate_up(gate, up, F, K, out);
}

}
