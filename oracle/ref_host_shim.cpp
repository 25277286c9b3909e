// ref_host_shim.cpp — C entry points over the reference's own host-only code
// (TEST INFRASTRUCTURE ONLY: built into oracle/_ref/ by oracle/build_ref.sh
// from the sources under /root/reference, and used by tests/ to pin the
// oracle's restatement of them).
//
//   CosineSchedule::lr_at     include/tensor/trainer/cosine_schedule.hpp:18-29
//   Dataset::load/next_batch  src/data/dataset.cpp:14-71
//
// The rest of the reference's step path is CUDA + cuBLAS and does not build
// here.
#include <cstdint>
#include <cstring>
#include <tensor/data/dataset.hpp>
#include <tensor/trainer/cosine_schedule.hpp>

extern "C" {

float ref_cosine_lr(float base_lr, int64_t warmup, int64_t total, float floor_frac,
                    int64_t step) {
    tensor::trainer::CosineSchedule s{base_lr, (std::size_t)warmup, (std::size_t)total,
                                      floor_frac};
    return s.lr_at((std::size_t)step);
}

// Loads `path` (a .bin file or a directory of them) and draws n_batches
// batches of B x T; inputs/targets receive n_batches * B * T ids each.
// Returns the total token count, or -1 if loading failed.
int64_t ref_dataset_batches(const char* path, int B, int T, int n_batches, int32_t* inputs,
                            int32_t* targets) {
    try {
        auto ds = tensor::data::Dataset::load(path);
        for (int i = 0; i < n_batches; i++) {
            auto [in, tg] = ds.next_batch(B, T);
            std::memcpy(inputs + (size_t)i * B * T, in.data(), in.size() * sizeof(int32_t));
            std::memcpy(targets + (size_t)i * B * T, tg.data(), tg.size() * sizeof(int32_t));
        }
        return (int64_t)ds.total_tokens();
    } catch (...) {
        return -1;
    }
}

}  // extern "C"
