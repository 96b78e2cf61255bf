// synth_gguf — writes one of the synthetic benchmark/test models.
//   synth_gguf <preset> <out.gguf> [-v] [--vocab [--eot-id N]]
//   synth_gguf --list
#include "synth_model.hpp"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "--list") == 0) {
        for (const auto& n : orc::synth_preset_names()) std::printf("%s\n", n.c_str());
        return 0;
    }
    if (argc < 3) {
        std::fprintf(stderr, "usage: synth_gguf <preset> <out.gguf> [-v] [--vocab [--eot-id N]] | --list\n");
        return 2;
    }
    orc::SynthSpec s;
    if (!orc::synth_preset(argv[1], s)) {
        std::fprintf(stderr, "unknown preset '%s'\n", argv[1]);
        return 2;
    }
    bool verbose = false;
    for (int i = 3; i < argc; ++i) {
        if (std::strcmp(argv[i], "-v") == 0) verbose = true;
        else if (std::strcmp(argv[i], "--vocab") == 0) s.vocab_stub = true;
        else if (std::strcmp(argv[i], "--eot-id") == 0 && i + 1 < argc) s.eot_id = std::atoi(argv[++i]);
        else {
            std::fprintf(stderr, "unknown option %s\n", argv[i]);
            return 2;
        }
    }
    auto t0 = std::chrono::steady_clock::now();
    std::string tmp = std::string(argv[2]) + ".partial";
    if (!orc::synth_write(s, tmp, verbose) || std::rename(tmp.c_str(), argv[2]) != 0) {
        std::fprintf(stderr, "synth_gguf: writing %s failed\n", argv[2]);
        std::remove(tmp.c_str());
        return 1;
    }
    double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    std::fprintf(stderr, "synth_gguf: %s -> %s (%.1f s)\n", argv[1], argv[2], dt);
    return 0;
}
