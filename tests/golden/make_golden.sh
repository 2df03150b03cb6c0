#!/bin/sh
# Regenerates tests/golden/data/ from the real reference.  Dev container only:
# needs /root/reference (the reference sources) and gcc.
#   tests/golden/make_golden.sh [quick]
set -e
cd "$(dirname "$0")/../.."
REF=${REF:-/root/reference}
make -C oracle ref REF="$REF"
mkdir -p oracle/_ref tests/golden/data
gcc -std=gnu11 -O2 -include stdint.h -I"$REF/include" -I"$REF/src" -w \
    tests/golden/gen_golden.c -o oracle/_ref/gen_golden \
    -Loracle/_ref -ldnnref -Wl,-rpath,"$PWD/oracle/_ref" -lm
OMP_NUM_THREADS=1 ./oracle/_ref/gen_golden "$@"
gcc -std=gnu11 -O2 -include stdint.h -I"$REF/include" -I"$REF/src" -w \
    tests/golden/gen_vlm.c -o oracle/_ref/gen_vlm \
    -Loracle/_ref -ldnnref -Wl,-rpath,"$PWD/oracle/_ref" -lm
OMP_NUM_THREADS=1 ./oracle/_ref/gen_vlm
gcc -std=gnu11 -O2 -include stdint.h -I"$REF/include" -I"$REF/src" -w \
    tests/golden/gen_ckpt.c -o oracle/_ref/gen_ckpt \
    -Loracle/_ref -ldnnref -Wl,-rpath,"$PWD/oracle/_ref" -lm
OMP_NUM_THREADS=1 ./oracle/_ref/gen_ckpt
# op- and layer-level fixtures: tests/c/ops_main.c is a caller of the public API
# only, built here against the reference and in tests/test_ops_gpu.py against
# include/dnn + libdnn_amd.so
gcc -std=gnu11 -O2 -include stdint.h -I"$REF/include" -I"$REF/src" -w \
    tests/c/ops_main.c -o oracle/_ref/ops_main \
    -Loracle/_ref -ldnnref -Wl,-rpath,"$PWD/oracle/_ref" -lm
mkdir -p tests/golden/data/ops
OMP_NUM_THREADS=1 ./oracle/_ref/ops_main tests/golden/data/ops
# sampled generation (temperature > 0): the reference's ids and each draw's
# distance to its CDF interval's edges
gcc -std=gnu11 -O2 -include stdint.h -I"$REF/include" -I"$REF/src" -w \
    tests/golden/gen_sample.c -o oracle/_ref/gen_sample \
    -Loracle/_ref -ldnnref -Wl,-rpath,"$PWD/oracle/_ref" -lm
OMP_NUM_THREADS=1 ./oracle/_ref/gen_sample
# the byte tokenizer: tests/c/tok_main.c against the reference
gcc -std=gnu11 -O2 -include stdint.h -I"$REF/include" -I"$REF/src" -w \
    tests/c/tok_main.c -o oracle/_ref/tok_main -Loracle/_ref -ldnnref -Wl,-rpath,"$PWD/oracle/_ref" -lm
./oracle/_ref/tok_main > tests/golden/data/tokenizer.json
