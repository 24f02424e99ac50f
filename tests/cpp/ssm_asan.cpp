// The .ssm reader and writer (lite_ssm_amd/csrc/ssm_file.hip) built with
// AddressSanitizer and UndefinedBehaviorSanitizer on the host, driven over
// files given on the command line (tests/test_ssm_asan.py makes corrupted
// and randomly mutated ones).  Every file is opened; an accepted file has its
// header, every index entry, every name lookup and the model lookups
// exercised, then it is closed.  One line per file on stdout:
//   opened <path> <n_tensors>
//   rejected <path>\t<message>
// With --write <path>, a small random-init model is written first (the
// writer and quantizer under the sanitizers), then read back the same way.
// Host code only: nothing here touches a GPU.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "lssm.h"

static int walk(const char* path) {
    lssm_ssm* f = nullptr;
    if (lssm_ssm_open(&f, path) != LSSM_OK) {
        std::printf("rejected %s\t%s\n", path, lssm_last_error());
        return 0;
    }
    lssm_ssm_header h{};
    if (lssm_ssm_get_header(f, &h) != LSSM_OK) {
        std::printf("error %s\tget_header: %s\n", path, lssm_last_error());
        lssm_ssm_close(f);
        return 1;
    }
    uint64_t bytes = 0;
    for (uint32_t i = 0; i < h.n_tensors; ++i) {
        char name[512];
        lssm_ssm_tensor t{}, u{};
        if (lssm_ssm_tensor_at(f, i, name, sizeof name, &t) != LSSM_OK) continue;   // name too long
        // (a name with a NUL byte in it is cut short as a C string, so the
        // lookup may miss it or find a shorter name)
        if (lssm_ssm_find(f, name, &u) != LSSM_OK && std::strlen(name) == 0) continue;
        // touch the payload's first and last byte inside the mapping
        if (t.nbytes) bytes += static_cast<const unsigned char*>(t.host)[0] +
                               static_cast<const unsigned char*>(t.host)[t.nbytes - 1];
    }
    lssm_ssm_tensor missing{};
    (void)lssm_ssm_find(f, "no.such.tensor", &missing);
    // the model lookups compute addresses only (device_base is never read)
    lssm_model_config cfg{};
    const void *embed = nullptr, *norm_f = nullptr, *lm_head = nullptr;
    std::vector<lssm_layer_weights> layers(64);
    (void)lssm_ssm_model(f, reinterpret_cast<const void*>(uintptr_t{1} << 40), &cfg, &embed, &norm_f, &lm_head,
                         layers.data(), (uint32_t)layers.size());
    lssm_ssm_close(f);
    std::printf("opened %s %u %llu\n", path, h.n_tensors, (unsigned long long)(bytes & 1));
    return 0;
}

int main(int argc, char** argv) {
    int i = 1, rc = 0;
    if (argc > 2 && std::strcmp(argv[1], "--write") == 0) {
        // 2 layers, d_model 64, expand 2, 2 heads x 64, d_state 32, vocab 96
        lssm_model_config cfg{64, 2, 32, 4, 2, 96, 2, 64, 64, 1, LSSM_BF16, LSSM_W_Q4_G64};
        if (lssm_ssm_write_random(argv[2], &cfg, 7) != LSSM_OK) {
            std::printf("error %s\twrite_random: %s\n", argv[2], lssm_last_error());
            return 1;
        }
        rc |= walk(argv[2]);
        i = 3;
    }
    for (; i < argc; ++i) rc |= walk(argv[i]);
    return rc;
}
