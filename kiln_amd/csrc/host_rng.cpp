// Host-side seeded normal noise, bit-compatible with torch.manual_seed(seed); torch.randn(n) on the CPU: the
// reference's torch_randn (engine/src/pipeline.cu:17-64), which draws the sampler's initial noise on the host
// (pipeline.cu:428-429) and copies it to the device.
//
// MT19937 (Matsumoto & Nishimura 1998) seeded with the low 32 bits of the seed; a 24-bit uniform per draw,
// (r & 0xffffff) * 2^-24; then Box-Muller over blocks of 16 values: for j < 8, u1 = 1 - d[j], u2 = d[j + 8],
// d[j] = sqrt(-2 ln u1) cos(2 pi u2), d[j + 8] = sqrt(-2 ln u1) sin(2 pi u2). A ragged tail (n % 16 != 0)
// draws 16 fresh uniforms for the last 16 values and transforms them again. n >= 16.
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace kiln {
namespace {

class Mt19937 {
   public:
    explicit Mt19937(uint32_t seed) : state_(624), next_(624) {
        state_[0] = seed;
        for (uint32_t i = 1; i < 624; i++) state_[i] = 1812433253u * (state_[i - 1] ^ (state_[i - 1] >> 30)) + i;
    }
    uint32_t operator()() {
        if (next_ == 624) twist();
        uint32_t y = state_[next_++];
        y ^= y >> 11;
        y ^= (y << 7) & 0x9d2c5680u;
        y ^= (y << 15) & 0xefc60000u;
        return y ^ (y >> 18);
    }
    float uniform24() { return (float)((*this)() & 0xffffffu) * (1.0f / 16777216.0f); }

   private:
    void twist() {
        for (int i = 0; i < 624; i++) {
            const uint32_t y = (state_[i] & 0x80000000u) | (state_[(i + 1) % 624] & 0x7fffffffu);
            state_[i] = state_[(i + 397) % 624] ^ (y >> 1) ^ (0x9908b0dfu & (0u - (y & 1u)));
        }
        next_ = 0;
    }
    std::vector<uint32_t> state_;
    int next_;
};

void box_muller16(float* d) {
    for (int j = 0; j < 8; j++) {
        const float r = sqrtf(-2.0f * logf(1.0f - d[j]));
        const float a = 6.28318530717958647692f * d[j + 8];
        d[j] = r * cosf(a);
        d[j + 8] = r * sinf(a);
    }
}

}  // namespace

bool host_torch_randn(float* out, uint64_t seed, size_t n) {
    if (n < 16) return false;
    Mt19937 g((uint32_t)(seed & 0xffffffffu));
    for (size_t i = 0; i < n; i++) out[i] = g.uniform24();
    for (size_t i = 0; i + 16 <= n; i += 16) box_muller16(out + i);
    if (n % 16) {
        float* t = out + n - 16;
        for (int i = 0; i < 16; i++) t[i] = g.uniform24();
        box_muller16(t);
    }
    return true;
}

}  // namespace kiln
