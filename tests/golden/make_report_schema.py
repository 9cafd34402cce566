"""Extracts the field names, in declaration order, of the reference's benchmark
report structs (crates/objeta-cuda/src/bin/bench_qgemv.rs, bench_selected_moe.rs,
crates/objeta-cuda/src/quant.rs, moe.rs) into report_schema.json. Run in a
container that holds the reference at /root/reference; the JSON it writes is the
committed fixture."""
import json
import os
import re

REF = "/root/reference/crates/objeta-cuda/src"
STRUCTS = {
    "bin/bench_qgemv.rs": ["QGemvStats", "QGemvStatsTelemetry", "QGemvStatsReport"],
    "bin/bench_selected_moe.rs": ["MoeStats", "MoeStatsTelemetry", "MoeStatsReport"],
    "quant.rs": ["QGemvNumerics", "QGemvNumericsSuite"],
    "moe.rs": ["MoeTelemetry", "BytesByTensorKind"],
}


def fields(src: str, name: str):
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\n\}", src, re.S)
    if not m:
        raise SystemExit(f"struct {name} not found")
    return re.findall(r"pub\s+(\w+)\s*:", m.group(1))


def main():
    out = {}
    for rel, names in STRUCTS.items():
        src = open(os.path.join(REF, rel)).read()
        for n in names:
            out[n] = fields(src, n)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "report_schema.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
