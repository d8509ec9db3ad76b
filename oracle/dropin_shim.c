/* Test infrastructure: backend/hip's table inside the reference's own
 * library, as the drop-in tests build it (oracle/Makefile, _ref/dropin_cli).
 *
 * The drop-in's needs are "hip" (libpktito_amd/backend_hip/kernels.c), which
 * a libpktito checkout with the hip backend answers by one more line in
 * core/os.c's pk_os_cpu_lacks: "hip" is met when pk_hip_init() opens the
 * device. The reference sources are
 * compiled here unedited, so the harness links with --wrap=pk_os_cpu_lacks
 * and answers it in this wrapper instead, every other need going to the
 * reference's own function (core/os.c:905-911). */
#include "pk_hip.h"

#include <string.h>

const char *__real_pk_os_cpu_lacks(const char *const *needs);

const char *__wrap_pk_os_cpu_lacks(const char *const *needs) {
    for (; *needs; needs++) {
        if (!strcmp(*needs, "hip")) {
            if (pk_hip_init() != PK_HIP_OK)
                return *needs;
            continue;
        }
        const char *one[2] = { *needs, NULL };
        const char *lack = __real_pk_os_cpu_lacks(one);
        if (lack)
            return lack;
    }
    return NULL;
}
