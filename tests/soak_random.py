"""On-demand randomised GPU parity sweep (not collected by pytest): more random cases of
the shapes test_gpu_random.py covers, with the same bit-exact checks against the oracle.

    python3 tests/soak_random.py N_CROSS N_GROUP SEED

draws N_CROSS cross-edge cases (d from 3 to 768, k from 1 to 64) and N_GROUP group-kNN
cases (d from 7 to 519, K from 1 to 64) from SEED and stops at the first mismatch."""
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE), HERE, os.path.join(os.path.dirname(HERE), "oracle")]

import filtervectorcode_refactor_amd as F  # noqa: E402
import test_gpu_random as T  # noqa: E402
from oracle import Oracle  # noqa: E402


def main():
    ncross, ngroup, base = (int(a) for a in sys.argv[1:4])
    ctx = F.HipContext(0)
    orc = Oracle()
    cross = T._cases(ncross, [3, 5, 17, 24, 31, 32, 33, 48, 64, 96, 127, 128, 129, 160, 200, 256, 300, 384, 520, 768],
                     [1, 2, 3, 6, 7, 8, 9, 12, 16, 17, 20, 32, 33, 40, 63, 64], base)
    group = T._cases(ngroup, [7, 16, 33, 40, 96, 127, 128, 129, 192, 256, 261, 300, 384, 519],
                     [1, 2, 5, 6, 10, 20, 31, 32, 33, 45, 50, 64], base + 1)
    t0 = time.time()
    for s, d, k, integer in cross:
        T.test_random_cross(ctx, orc, base * 1000 + s, d, k, integer)
    print(f"cross: {len(cross)} cases bit-exact ({time.time() - t0:.0f} s)", flush=True)
    t0 = time.time()
    for s, d, k, integer in group:
        T.test_random_group_knn(ctx, orc, base * 1000 + s, d, k, integer)
    print(f"group kNN: {len(group)} cases bit-exact ({time.time() - t0:.0f} s)", flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
