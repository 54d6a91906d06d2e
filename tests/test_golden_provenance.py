"""Provenance of tests/golden/reference_digests.json: every digest recorded
there appears in the reference file its `source` names (an evidence record
docs/results/*.json, or the Rust test holding a known answer; "same record"
refers to the previous section's record).  Files are read as text.  Runs where
the reference checkout is present (the build container); skipped elsewhere."""
import json
import os
import re

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("LOOM_REFERENCE_ROOT", "/root/reference")
GOLDEN = json.load(open(os.path.join(HERE, "golden", "reference_digests.json")))

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "docs", "results")),
                                reason="reference checkout not present")


def _entries():
    """(section, source file, [digest strings]) for every sourced section."""
    out = []
    prev = None
    for key, sec in GOLDEN.items():
        if not isinstance(sec, dict) or "source" not in sec:
            continue
        src = prev if sec["source"].startswith("same record") else sec["source"].split()[0]
        src = src.split(":")[0]
        prev = src
        text = json.dumps(sec)
        digests = sorted(set(re.findall(r'"([0-9a-f]{16})"', text)))
        out.append((key, src, digests))
    return out


@pytest.mark.parametrize("key,src,digests", _entries(), ids=[e[0] for e in _entries()])
def test_digests_appear_in_their_source_record(key, src, digests):
    record = open(os.path.join(REF, src)).read()
    if src.endswith(".json"):
        json.loads(record)  # a data record
    else:
        record = record.replace("_", "").lower()  # Rust hex literals: 0xf25b_8807_...
    missing = [d for d in digests if d not in record]
    assert not missing, f"{key}: digests not in {src}: {missing}"
