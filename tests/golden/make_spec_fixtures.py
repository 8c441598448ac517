"""Builds tests/golden/spec_fixtures.json from the reference's own data files:
the serde KernelSpec documents and the binding manifest its `emit-suite`
command wrote (reports/generated-native/manifest.json, *.json) and the example
specs (examples/kernels/*.json). Only data is kept (spec, bindings); no
reference source text. Run in the build container, where /root/reference exists.
"""
import glob
import json
import os

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    manifest = json.load(open(os.path.join(REF, "reports/generated-native/manifest.json")))
    cases = []
    for entry in manifest["cases"]:
        spec_file = os.path.join(REF, "reports/generated-native", entry["case"] + ".json")
        cases.append({
            "case": entry["case"],
            "spec": entry["spec"],
            "spec_file_text": open(spec_file).read(),
            "bindings": entry["bindings"],
            "reference_launch": entry["launch"],
        })
    examples = []
    for path in sorted(glob.glob(os.path.join(REF, "examples/kernels/*.json"))):
        examples.append({"file": os.path.basename(path), "text": open(path).read()})
    out = {
        "source": "reports/generated-native/manifest.json (schema_version %s), reports/generated-native/*.json, "
                  "examples/kernels/*.json" % manifest.get("schema_version"),
        "cases": cases,
        "examples": examples,
    }
    with open(os.path.join(HERE, "spec_fixtures.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
