// Build driver for oracle/_ref: exposes the reference's own host-callable RNG
// header (src/nanorts/core/cuda/conflict_draw.cuh, compiled from where it lies
// under the reference checkout) through a C ABI, so the oracle's threefry,
// fold_in, randint and CANCEL_RANDOM draws can be compared with it.
// TEST INFRASTRUCTURE ONLY.  hipcc supplies the __host__/__device__
// attributes the header uses; nothing of the header is copied here.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "conflict_draw.cuh"

extern "C" {

void ref_threefry2x32(const uint32_t key[2], uint32_t x[2]) {
    nanorts::draws::threefry2x32(nanorts::draws::Key{key[0], key[1]}, x[0], x[1]);
}

void ref_fold_in(const uint32_t key[2], int32_t data, uint32_t out[2]) {
    const nanorts::draws::Key k = nanorts::draws::fold_in(nanorts::draws::Key{key[0], key[1]}, data);
    out[0] = k.k0;
    out[1] = k.k1;
}

int32_t ref_randint01(const uint32_t key[2]) {
    return nanorts::draws::randint01(nanorts::draws::Key{key[0], key[1]});
}

int32_t ref_conflict_draw(const uint32_t root[2], int32_t time, int32_t birth, int32_t ordinal) {
    const nanorts::draws::Key address = nanorts::draws::conflict_address(nanorts::draws::Key{root[0], root[1]}, time, birth);
    return nanorts::draws::conflict_draw(address, ordinal);
}
}
