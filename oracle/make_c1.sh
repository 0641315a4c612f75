#!/bin/sh
# make_c1.sh - TEST INFRASTRUCTURE ONLY: the 4-layer synthetic model (D 512,
# 8/2 heads x 64, 32 experts top-4, expert width 256, one shared expert,
# vocabulary 4096, seed 1) written by the reference's own tools (built from
# its sources by `make -C oracle tools`) into oracle/_ref/c1:
#   src/            tlmc synth output (model.safetensors, config.json)
#   c1.tlmm, d0/    tlmc compile --profile exact on one drive directory
#   bench.txt       tierlm bench --prompt-len 64 -n 64 (the greedy tokens)
# and the SHA-256 of the synth output checked against the values recorded when
# the reference was surveyed.  Nothing here is copied from the reference.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
B="$HERE/_ref/bin"
O="$HERE/_ref/c1"
[ -x "$B/tlmc" ] && [ -x "$B/tierlm" ] || make -C "$HERE" tools >/dev/null
rm -rf "$O"
mkdir -p "$O/d0"
"$B/tlmc" synth --out "$O/src" --layers 4 --d-model 512 --heads 8 --kv-heads 2 --head-dim 64 \
    --experts 32 --top-k 4 --d-expert 256 --shared 1 --vocab 4096 --seed 1 > "$O/synth.log" 2>&1
echo "22b9ee2eb5c15c0c73ec8cd931e1b723bec27c675b08e35375b62910dd84f651  $O/src/model.safetensors" | sha256sum -c -
echo "e14365572c6d294aef224ab6f6900f6b69ae4989628779a5a1cb608358278a3d  $O/src/config.json" | sha256sum -c -
"$B/tlmc" compile "$O/src" --out "$O/c1.tlmm" --drives "$O/d0" --profile exact > "$O/compile.log" 2>&1
# only the compiled store travels with the tree: drop the f32 source and the
# compiler's scratch
rm -rf "$O/src" "$O/c1.work"
