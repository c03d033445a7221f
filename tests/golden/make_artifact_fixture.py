"""Write tests/golden/reference_artifact/ with the reference's own artifact
writer (src/nanoquant/runtime/packed_artifact.py:306-372) and packer
(src/nanoquant/runtime/packed.py:393-411).

Run in the build container only, where the reference checkout is readable:
    python tests/golden/make_artifact_fixture.py
It imports the reference package from /root/reference/src. The committed
output is data (a manifest and two safetensors shards); nothing from the
reference travels with it. The layers come from ``artifact_recipe.py``.
"""

from __future__ import annotations

import shutil
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE_SRC = Path("/root/reference/src")
OUTPUT = HERE / "reference_artifact"


def main() -> None:
    sys.path.insert(0, str(REFERENCE_SRC))
    sys.path.insert(0, str(HERE))
    from artifact_recipe import BLOCKS, dense_layer
    from nanoquant.runtime.artifact import RuntimeModelMetadata
    from nanoquant.runtime.backend import QuantizedLinearSpec
    from nanoquant.runtime.logical import LogicalLayerState
    from nanoquant.runtime.packed import pack_logical_layer
    from nanoquant.runtime.packed_artifact import write_packed_artifact

    def state(index: int):
        kwargs = dense_layer(index)
        spec = QuantizedLinearSpec(**kwargs.pop("spec_args"))
        return pack_logical_layer(LogicalLayerState(spec, **kwargs))

    blocks = {block: [state(i) for i in members] for block, members in BLOCKS.items()}
    if OUTPUT.exists():
        shutil.rmtree(OUTPUT)
    metadata = RuntimeModelMetadata("fixture/nanoquant-amd", "r1", "qwen3", "config-hash", "tokenizer-hash")
    written = write_packed_artifact(OUTPUT, metadata, "0" * 64, blocks)
    print(f"wrote {written.root}: {written.manifest.layer_count} layers, {written.manifest.weight_bytes} bytes")


if __name__ == "__main__":
    main()
