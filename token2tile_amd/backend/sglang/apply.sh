#!/usr/bin/env bash
# Registers the Token2Tile attention backend (MI355X / gfx950) in an SGLang
# checkout at the commit the patch was written against:
#   apply.sh <sglang checkout> [--check]
# The patch adds the T2T_ATTN enum member and its list entries, the
# denoising-stage metadata branch and the MiniMax-H3 layout record, each
# calling token2tile_amd.backend.sglang_hooks.  The ROCm resolver is added to
# SGLang's ROCm platform module by hand (a few lines, shown in the
# integration notes), because its resolver table is platform code this patch
# does not see.  token2tile_amd must be importable by SGLang's Python.
set -euo pipefail
here=$(cd "$(dirname "$0")" && pwd)
sgl=${1:?usage: apply.sh <sglang checkout> [--check]}
base=880ab72f34ead8f39544c7c7e08edbd443964a1f
head=$(git -C "$sgl" rev-parse HEAD)
if [ "$head" != "$base" ]; then
  echo "expected SGLang at $base, found $head" >&2
  exit 1
fi
git -C "$sgl" apply --check "$here/token2tile_rocm.patch"
if [ "${2:-}" = "--check" ]; then
  echo "patch applies cleanly"
  exit 0
fi
git -C "$sgl" apply "$here/token2tile_rocm.patch"
python3 - <<'PY'
import token2tile_amd.backend.sglang_hooks as h
print("Token2Tile backend hooks:", h.BACKEND_PATH, "- now add the ROCm resolver "
      "(resolve_backend) to SGLang's ROCm platform and select attention_backend=t2t_attn")
PY
