// Compiles the reference-named C++ drop-ins of lutmac_hip_compat.h against a
// PackedTensor-shaped struct and runs lut_linear / int4_gemv / precompute_luts
// on host buffers, the way model.cpp and tests/test_lut_gemm.cpp call them in
// the LutMac tree.  Prints one line per check and exits non-zero on failure.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "lutmac_hip_compat.h"

namespace {

struct Blk68 { uint8_t b[68]; };
struct Blk36 { uint8_t b[36]; };
struct Blk72 { uint8_t b[72]; };
struct Blk100 { uint8_t b[100]; };
struct Blk132 { uint8_t b[132]; };
struct Blk160 { uint8_t b[164]; };
struct Blk192 { uint8_t b[196]; };
struct Blk260 { uint8_t b[260]; };

// Same member names as lutmac::PackedTensor (types.hpp:470-492).
struct FakePackedTensor {
  std::string name;
  std::vector<size_t> shape;
  std::vector<Blk68> blocks;
  std::vector<Blk72> int2_blocks;
  std::vector<Blk100> int3_blocks;
  std::vector<Blk132> int4_blocks;
  std::vector<Blk160> int5_blocks;
  std::vector<Blk192> int6_blocks;
  std::vector<Blk36> binary_blocks;
  std::vector<Blk260> int8_blocks;
  std::vector<float> raw_data;
  float global_scale = 1.0f;
  bool is_quantized = true;
  int quant_bits = 4;
};

int failures = 0;
void report(const char *name, bool ok, double got, double want) {
  std::printf("%s %s: got %.6f want %.6f\n", ok ? "PASS" : "FAIL", name, got, want);
  if (!ok) ++failures;
}

}  // namespace

int main() {
  // test_lut_gemm.cpp:218-260 restated: ramp (i%15)-7 at scale 0.5, x = 1.
  {
    FakePackedTensor w;
    w.shape = {1, 32};
    w.quant_bits = 4;
    w.int4_blocks.resize(1);
    uint8_t q[256];
    for (int i = 0; i < 256; ++i) q[i] = i < 32 ? uint8_t((i % 15) - 7 + 8) : 8;
    for (int i = 0; i < 128; ++i) w.int4_blocks[0].b[i] = uint8_t((q[2 * i] << 4) | q[2 * i + 1]);
    const float s = 0.5f;
    std::memcpy(w.int4_blocks[0].b + 128, &s, 4);
    std::vector<float> x(32, 1.0f), y(1, 0.0f);
    lutmac_hip::lut_linear(w, nullptr, x.data(), y.data());
    report("int4 ramp (lut_linear)", std::fabs(y[0] + 6.5f) < 0.01f, y[0], -6.5);
    std::vector<float> xp(256, 0.0f);
    for (int i = 0; i < 32; ++i) xp[i] = 1.0f;
    lutmac_hip::int4_gemv(w.int4_blocks.data(), 1, xp.data(), y.data(), 1, 32);
    report("int4 ramp (int4_gemv)", std::fabs(y[0] + 6.5f) < 0.01f, y[0], -6.5);
  }
  // test_lut_gemm.cpp:135-165 restated: ternary +1 weights, x = [1,2,3,4] -> 10.
  {
    FakePackedTensor w;
    w.shape = {1, 4};
    w.quant_bits = 2;
    w.blocks.resize(1);
    std::memset(w.blocks[0].b, 0, 68);
    std::memset(w.blocks[0].b + 32, 0xFF, 32);
    w.blocks[0].b[32] = 0x0F;
    const float s = 1.0f;
    std::memcpy(w.blocks[0].b + 64, &s, 4);
    // lut_linear rotates ternary activations, so feed FWHT^-1(x) = FWHT(x).
    std::vector<float> x(256, 0.0f);
    x[0] = 1, x[1] = 2, x[2] = 3, x[3] = 4;
    std::vector<float> xr = x;
    lutmac_hip::apply_hadamard_rotation(xr.data(), 256);
    std::vector<float> y(1, 0.0f);
    lutmac_hip::lut_gemv(w.blocks.data(), 1, x.data(), y.data(), 1, 4);
    report("ternary all-ones (lut_gemv)", y[0] == 10.0f, y[0], 10.0);
  }
  // test_lut_gemm.cpp:17-55 restated: tables of [1,2,3,4].
  {
    const float a[4] = {1, 2, 3, 4};
    float t[16];
    lutmac_hip::precompute_luts(a, 4, t);
    const float want[16] = {0, 4, 3, 7, 2, 6, 5, 9, 1, 5, 4, 8, 3, 7, 6, 10};
    bool ok = true;
    for (int i = 0; i < 16; ++i) ok = ok && t[i] == want[i];
    report("precompute_luts KAT", ok, t[15], 10.0);
    float t1[16];
    lutmac_hip::precompute_lut(a, t1);   // one group (lut_gemm.hpp:30-44)
    ok = true;
    for (int i = 0; i < 16; ++i) ok = ok && t1[i] == want[i];
    report("precompute_lut KAT", ok, t1[15], 10.0);
  }
  // test_lut_gemm.cpp:57-88 restated: weights [+1, -1, 0, +1] -> pos 0b1001,
  // neg 0b0100; the same nibbles in group 1 (low nibble of byte 0).
  {
    const uint8_t sign[4] = {0b01000100, 0, 0, 0}, zero[4] = {0b00100010, 0, 0, 0};
    uint8_t pos = 0, neg = 0;
    lutmac_hip::extract_indices(sign, zero, 0, pos, neg);
    uint8_t pos1 = 0, neg1 = 0;
    lutmac_hip::extract_indices(sign, zero, 1, pos1, neg1);
    report("extract_indices KAT", pos == 0b1001 && neg == 0b0100 && pos1 == 0b1001 && neg1 == 0b0100, pos, 9.0);
  }
  std::printf("%d failure(s)\n", failures);
  return failures ? 1 : 0;
}
