// Host-only driver of the GGUF reader (host/hy_gguf.cpp) for an AddressSanitizer /
// UndefinedBehaviorSanitizer build: for every file named on the command line it opens
// the file through the C ABI and, when the open succeeds, reads every tensor's
// metadata, converts every tensor to f32 and reads a few keys.  Any result code is
// accepted; a sanitizer report or a crash is the failure.
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/hy_moe.h"
#include "../../hunyuan-image-3-80b.cpp_amd/host/hy_gguf.hpp"

namespace hy {
// the library's error slot (hy_capi.hip is not part of this host-only build)
int set_last_error(int code, const std::string&) { return code; }
const GgufFile& gguf_file(const hy_gguf* g);  // hy_gguf.cpp
}  // namespace hy

int main(int argc, char** argv) {
    int opened = 0;
    for (int i = 1; i < argc; i++) {
        hy_gguf* g = nullptr;
        if (hy_gguf_open(argv[i], &g) != HY_OK) continue;
        opened++;
        const hy::GgufFile& f = hy::gguf_file(g);
        for (const auto& t : f.tensors) {
            const std::string& name = t.name;
            int32_t type = 0;
            uint32_t nd = 0;
            uint64_t ne[4] = {0, 0, 0, 0};
            if (hy_gguf_tensor(g, name.c_str(), &type, &nd, ne, nullptr, nullptr) != HY_OK) continue;
            uint64_t n = 1;
            for (uint32_t d = 0; d < nd && d < 4; d++) n *= ne[d];
            if (n == 0 || n > (1u << 22)) continue;
            std::vector<float> out(n);
            (void)hy_gguf_tensor_f32(g, name.c_str(), out.data(), n);
        }
        uint32_t u = 0;
        float x = 0.f;
        (void)hy_gguf_get_u32(g, "hunyuan.hidden_size", &u);
        (void)hy_gguf_get_u32(g, "general.alignment", &u);
        (void)hy_gguf_get_f32(g, "hunyuan.rms_norm_eps", &x);
        hy_gguf_close(g);
    }
    std::printf("opened %d of %d files\n", opened, argc - 1);
    return 0;
}
