#!/bin/sh
# make_c6d.sh - TEST INFRASTRUCTURE ONLY: a synthetic model whose first two
# layers are dense FFNs (first_k_dense_replace = 2): 4 layers, D 512, 8 query /
# 2 key heads of width 64, qk-norm, dense FFN width 1024, then 16 experts top-4
# of width 256 with one shared expert of width 256 under the softmax router,
# vocabulary 2048, seed 21.  Written by the reference's own tools (built from
# its sources by `make -C oracle tools`) into oracle/_ref/c6d:
#   c6d.tlmm, d0/   tlmc compile --profile exact
# with the SHA-256 of the synth output checked against the values recorded
# when this fixture was first made.  Nothing here is copied from the reference.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
B="$HERE/_ref/bin"
O="$HERE/_ref/c6d"
[ -x "$B/tlmc" ] && [ -x "$B/tierlm" ] || make -C "$HERE" tools >/dev/null
rm -rf "$O"
mkdir -p "$O/d0"
"$B/tlmc" synth --out "$O/src" --layers 4 --d-model 512 --heads 8 --kv-heads 2 --head-dim 64 \
    --experts 16 --top-k 4 --d-expert 256 --shared 1 --vocab 2048 --seed 21 \
    --dense-layers 2 --dense-ffn 1024 > "$O/synth.log" 2>&1
echo "a21eb5934a630d113c0a13a20305e5db704b70b4b8166b4fbac0a0ca16541eb9  $O/src/model.safetensors" | sha256sum -c -
echo "20feac32c07b8fb973f4c87d9619e38c8dab2230343cb3d76a8722aef3f30dc2  $O/src/config.json" | sha256sum -c -
"$B/tlmc" compile "$O/src" --out "$O/c6d.tlmm" --drives "$O/d0" --profile exact > "$O/compile.log" 2>&1
rm -rf "$O/src" "$O/c6d.work"
