// When the GPU path can't run, llama.cpp must not see XDNA0 at all (the
// reference's tests/test-safe-start.cpp): the add-on still loads, but offers
// no device. The failing check is chosen by the command line:
//   (none)        GGML_XDNA_DEVICE names a GPU that does not exist
//   --host-only   GGML_XDNA_HOST_ONLY=1 (this backend has no CPU path)
//   --no-gpu      run as is on a machine without a GPU
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "mini_ggml.h"

int main(int argc, char ** argv) {
    const char * mode = argc > 1 ? argv[1] : "";
    unsetenv("GGML_XDNA_PLAN_ONLY");
    if (strcmp(mode, "--host-only") == 0) {
        setenv("GGML_XDNA_HOST_ONLY", "1", 1);
    } else if (strcmp(mode, "--no-gpu") != 0) {
        setenv("GGML_XDNA_DEVICE", "99", 1);
        unsetenv("GGML_XDNA_HOST_ONLY");
    }
    ggml_backend_load_all();
    test_check(ggml_backend_dev_count() >= 1 && ggml_backend_dev_by_type(GGML_BACKEND_DEVICE_TYPE_CPU) != nullptr,
               "the backend loads (GGML_BACKEND_PATH set) and the host device is there");
    test_check(ggml_backend_dev_by_name("XDNA0") == nullptr, "no XDNA0 device when the GPU path can't run (%s)",
               *mode ? mode : "no such GPU");
    printf("%s\n", test_failures() ? "FAILED" : "ALL PASS");
    return test_failures() ? 1 : 0;
}
