"""Writes tests/golden/golden.npz from the CPU oracle and the seeded cases.

    python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention_oracle as orc  # noqa: E402
from tests.golden import cases as C  # noqa: E402


def main():
    out = {}
    d = C.decode_case()
    kc, vc = d["kc"].clone(), d["vc"].clone()
    orc.paged_kv_append(kc, vc, d["kn"], d["vn"], d["bt"], d["pos"])
    out["decode_inputs_sha"] = np.array(C.digest(*d.values()))
    out["decode_pool_after_sha"] = np.array(C.digest(kc, vc))
    out["decode_out"] = orc.paged_decode(d["q"], kc, vc, d["bt"], d["pos"] + 1).numpy()

    p = C.prefill_case()
    out["prefill_inputs_sha"] = np.array(C.digest(p["q"], p["k"], p["v"], p["cu"]))
    out["prefill_out"] = orc.varlen_causal(p["q"], p["k"], p["v"], p["cu"]).numpy()

    r = C.rope_case()
    out["rope_inputs_sha"] = np.array(C.digest(r["x"], r["pos"], r["inv_freq"]))
    out["rope_out"] = orc.partial_rope(r["x"], r["pos"], r["inv_freq"], C.ROTARY).float().numpy()

    g = C.gate_case()
    out["gate_inputs_sha"] = np.array(C.digest(g["x"], g["gate"]))
    out["gate_out"] = orc.gate_pack(g["x"], g["gate"]).float().numpy()

    f = C.fill_case()
    kc, vc = f["kc"].clone(), f["vc"].clone()
    orc.paged_kv_fill_varlen(kc, vc, f["k"], f["v"], f["bt"], f["cu"])
    out["fill_inputs_sha"] = np.array(C.digest(f["k"], f["v"], f["kc"], f["vc"], f["bt"], f["cu"]))
    out["fill_pool_after_sha"] = np.array(C.digest(kc, vc))

    path = Path(__file__).with_name("golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
