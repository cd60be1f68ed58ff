"""Writes reference_workflow_nodes.json: the attention nodes of the reference's saved workflows.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_workflow_nodes.py /root/reference/workflows
For every node of the three ComfyUI workflow files whose type starts with
RDNA35 it records the node type, the saved widget values and the names of its
input and output sockets: the data a saved workflow binds to when ComfyUI
loads it against this package's node classes.
"""
from __future__ import annotations

import json
import pathlib
import sys


def extract(workflow_dir: pathlib.Path) -> dict:
    out = {}
    for path in sorted(workflow_dir.glob("*.json")):
        nodes = json.loads(path.read_text())["nodes"]
        rows = []
        for node in nodes:
            if not str(node.get("type", "")).startswith("RDNA35"):
                continue
            rows.append({"type": node["type"],
                         "widgets_values": node.get("widgets_values", []),
                         "inputs": [s["name"] for s in node.get("inputs", [])],
                         "outputs": [s["name"] for s in node.get("outputs", [])]})
        out[path.name] = rows
    return out


if __name__ == "__main__":
    src = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/workflows")
    dst = pathlib.Path(__file__).with_name("reference_workflow_nodes.json")
    dst.write_text(json.dumps(extract(src), indent=1) + "\n")
    print(f"wrote {dst}")
