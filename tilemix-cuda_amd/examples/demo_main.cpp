// TileMix demo on MI355X: the workload of the reference demo (src/main.cu:22-69)
// driven through the reference-compatible C++ API of include/attention_fused.h.
//
// M=1000 queries, N=1003 keys, d=128, routing groups of 2 key tiles with the
// alternating mask 0xaaaa... (odd groups INT8, even groups FP16).
//
// `tilemix_demo --rounds R` also times R more rounds of the two calls
// (quantize_tilemix_qk + launch_fused_fp16_attention) on the null stream with
// HIP events, after as many untimed ones, and prints the time per round.

#include "attention_fused.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace {

void ensure(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
    }
}

// Owning device allocation released on scope exit.
template <class T>
class Device {
public:
    explicit Device(std::size_t count) : count_(count) {
        ensure(hipMalloc(reinterpret_cast<void**>(&ptr_), count * sizeof(T)), "hipMalloc");
    }
    ~Device() { (void)hipFree(ptr_); }
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
    T* get() const { return ptr_; }
    void upload(const std::vector<T>& host) {
        ensure(hipMemcpy(ptr_, host.data(), count_ * sizeof(T), hipMemcpyHostToDevice), "upload");
    }

private:
    T* ptr_ = nullptr;
    std::size_t count_;
};

}  // namespace

int main(int argc, char** argv) {
    try {
        int rounds = 0;
        for (int a = 1; a < argc; ++a) {
            if (std::strcmp(argv[a], "--rounds") == 0 && a + 1 < argc) rounds = std::atoi(argv[++a]);
            else throw std::runtime_error(std::string("unknown argument: ") + argv[a]);
        }
        if (rounds < 0) throw std::runtime_error("--rounds takes a count >= 0");
        constexpr int M = 1000, N = 1003, d = 128, group = 2;
        const std::size_t q_count = static_cast<std::size_t>(M) * d;
        const std::size_t kv_count = static_cast<std::size_t>(N) * d;
        const std::size_t words = tilemix_routing_word_count(M, N, group);
        const std::size_t q_blocks = (M - 1) / kTileMixQQuantRows + 1;
        const std::size_t k_blocks = (N - 1) / kTileMixKQuantRows + 1;

        std::size_t free_bytes = 0, total_bytes = 0;
        ensure(hipMemGetInfo(&free_bytes, &total_bytes), "hipMemGetInfo");
        const std::size_t needed = 2 * (q_count + 2 * kv_count) + 4 * q_count + 8 * words + q_count +
                                   kv_count + 2 * (q_blocks + k_blocks);
        if (needed > free_bytes / 4) throw std::runtime_error("inputs exceed the device memory budget");

        // Deterministic periodic inputs (periods 17, 19 and 23 for Q, K and V).
        std::vector<__half> q(q_count), k(kv_count), v(kv_count);
        for (std::size_t i = 0; i < q_count; ++i) q[i] = __float2half(0.125f * static_cast<float>(static_cast<int>(i % 17) - 8));
        for (std::size_t i = 0; i < kv_count; ++i) k[i] = __float2half(0.125f * static_cast<float>(static_cast<int>(i % 19) - 9));
        for (std::size_t i = 0; i < kv_count; ++i) v[i] = __float2half(0.1f * static_cast<float>(static_cast<int>(i % 23) - 11));
        const std::vector<std::uint64_t> mask(words, UINT64_C(0xaaaaaaaaaaaaaaaa));

        Device<__half> dq(q_count), dk(kv_count), dv(kv_count);
        Device<float> out(q_count);
        Device<std::int8_t> q8(q_count), k8(kv_count);
        Device<__half> q_scales(q_blocks), k_scales(k_blocks);
        Device<std::uint64_t> mask_words(words);
        dq.upload(q);
        dk.upload(k);
        dv.upload(v);
        mask_words.upload(mask);

        ensure(quantize_tilemix_qk(dq.get(), dk.get(), q8.get(), k8.get(), q_scales.get(), k_scales.get(), M, N, d),
               "quantize_tilemix_qk");
        const TileMixRouting routing{mask_words.get(), words, group};
        const TileMixQuantized quantized{q8.get(), k8.get(), q_scales.get(), k_scales.get()};
        ensure(launch_fused_fp16_attention(dq.get(), dk.get(), dv.get(), out.get(), M, N, d,
                                           1.0f / std::sqrt(static_cast<float>(d)), nullptr, routing, quantized),
               "launch_fused_fp16_attention");
        ensure(hipDeviceSynchronize(), "hipDeviceSynchronize");
        std::vector<float> result(q_count);
        ensure(hipMemcpy(result.data(), out.get(), q_count * sizeof(float), hipMemcpyDeviceToHost), "download");
        std::printf("TileMix attention: M=%d N=%d d=%d output[0]=%.9g\n", M, N, d, result[0]);
        std::printf("Routing: %d key tiles/group, %zu packed words; bit 0=FP16, bit 1=INT8 MFMA\n", group, words);
        if (rounds > 0) {
            auto round = [&]() {
                ensure(quantize_tilemix_qk(dq.get(), dk.get(), q8.get(), k8.get(), q_scales.get(), k_scales.get(), M,
                                           N, d),
                       "quantize_tilemix_qk");
                ensure(launch_fused_fp16_attention(dq.get(), dk.get(), dv.get(), out.get(), M, N, d,
                                                   1.0f / std::sqrt(static_cast<float>(d)), nullptr, routing,
                                                   quantized),
                       "launch_fused_fp16_attention");
            };
            for (int r = 0; r < rounds; ++r) round();  // untimed: the clock rises under sustained work
            hipEvent_t start = nullptr, stop = nullptr;
            ensure(hipEventCreate(&start), "hipEventCreate");
            ensure(hipEventCreate(&stop), "hipEventCreate");
            ensure(hipEventRecord(start, nullptr), "hipEventRecord");
            for (int r = 0; r < rounds; ++r) round();
            ensure(hipEventRecord(stop, nullptr), "hipEventRecord");
            ensure(hipEventSynchronize(stop), "hipEventSynchronize");
            float ms = 0.0f;
            ensure(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
            (void)hipEventDestroy(start);
            (void)hipEventDestroy(stop);
            std::printf("Timed: %d rounds of quantize_tilemix_qk + launch_fused_fp16_attention, %.2f us per round\n",
                        rounds, 1000.0f * ms / static_cast<float>(rounds));
        }
        return 0;
    } catch (const std::exception& error) {
        std::fprintf(stderr, "ERROR: %s\n", error.what());
        return 1;
    }
}
