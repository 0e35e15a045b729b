"""Copy the reference's own fixture rows for this path into tests/golden/.

Run here (where /root/reference exists); the GPU box only reads the committed
JSON.  Sources:
  - quant/testdata/oq.json "tensor_bytes", the fixture of
    TestTensorQuantizedBytesParity (quant/oq_test.go:158-165);
  - compute/testdata/deepseek_args.json "routing", the fixture of
    TestDeepseekV3GroupExpertSelectParity (compute/models/deepseekv3_test.go:130-163);
  - compute/testdata/safetensors_header.json, the container blobs and parsed
    truth of TestParseSafetensorsHeaderParity (compute/safetensors_test.go:29-94);
  - compute/testdata/loader_tensors.json, the blob and per-tensor bytes of
    TestTensorBytesParity / TestLoadTensorsParity (compute/loader_test.go:43-112).
"""
import json
import os
import sys

REF = os.environ.get("FMXQ_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> int:
    src = os.path.join(REF, "quant", "testdata", "oq.json")
    with open(src) as f:
        data = json.load(f)
    out = {"source": "quant/testdata/oq.json#tensor_bytes", "tensor_bytes": data["tensor_bytes"]}
    with open(os.path.join(HERE, "oq_tensor_bytes.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    with open(os.path.join(REF, "compute", "testdata", "deepseek_args.json")) as f:
        routing = json.load(f)["routing"]
    out = {"source": "compute/testdata/deepseek_args.json#routing", "routing": routing}
    with open(os.path.join(HERE, "deepseek_routing.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    for name in ("safetensors_header.json", "loader_tensors.json"):
        with open(os.path.join(REF, "compute", "testdata", name)) as f:
            data = json.load(f)
        out = {"source": "compute/testdata/" + name, "data": data}
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(out, f, indent=1)
            f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
