"""Write tests/golden/block_traces.json from the reference's own Python source.

Run only where the reference tree is present (the tests read the committed
JSON, never the reference):  python tests/golden/make_block_traces.py

It imports the reference's pure-Python BlockManager, MiniScheduler,
EngineCore, Sequence and SamplingParams (they import torch, math and
dataclasses only) and drives them with tests/golden/trace_driver.py.  Only the
recorded input/output vectors are committed; no reference code is copied.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE_SRC = Path("/root/reference/src")


def main() -> None:
    sys.path.insert(0, str(REFERENCE_SRC))
    sys.path.insert(0, str(HERE))
    import torch
    from nanovllm_ascend.engine import EngineCore
    from nanovllm_ascend.npu.block_manager import BlockManager
    from nanovllm_ascend.sampling_params import SamplingParams
    from nanovllm_ascend.scheduler import MiniScheduler
    from nanovllm_ascend.sequence import Sequence

    import trace_driver

    out = {}
    for name in trace_driver.SCENARIOS:
        out[name] = trace_driver.run_scenario(
            name, BlockManager=BlockManager, MiniScheduler=MiniScheduler, EngineCore=EngineCore,
            Sequence=Sequence, SamplingParams=SamplingParams, torch_mod=torch)
        print(f"{name}: {len(out[name])} events")
    (HERE / "block_traces.json").write_text(json.dumps(out, separators=(",", ":")))


if __name__ == "__main__":
    main()
