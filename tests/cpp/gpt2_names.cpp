// Test driver (built and run by tests/test_gpt2_weights.py on the CPU): for each argument, the kael
// name the library's checkpoint reader gives a stored GPT-2 tensor name, and whether kael keeps that
// weight transposed ("<kael name> <0|1>" per line).
#include <cstdio>

#include "kd_safetensors.h"

int main(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        const std::string name = kd::safetensors::translated_gpt2_name(argv[i]);
        std::printf("%s %d\n", name.c_str(), kd::safetensors::stored_transposed(name) ? 1 : 0);
    }
    return 0;
}
