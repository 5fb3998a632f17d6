"""Summaries of rocprofv3 counter CSVs (``-f csv``) for the decode kernels.

HBM traffic per decode launch, after two counter runs of ``bench.py
--copy-calibration``, one with ``--pmc FETCH_SIZE`` and one with ``--pmc
WRITE_SIZE``:

    python -m qwen_megakernel.counters FETCH.csv WRITE.csv --timed 1024

``FETCH_SIZE`` / ``WRITE_SIZE`` are in KiB per dispatch.  Each counter is
scaled by the ratio of the known size of the calibration copy (1 GiB read and
1 GiB written) to what the same counter reads for that copy, then averaged
over the last ``--timed`` decode dispatches (the timed region of the run).

Shader-sequencer counters per kernel (any ``SQ_*`` / ``GRBM_*`` set):

    python -m qwen_megakernel.counters sq A.csv [B.csv ...] --timed 256

gives, for every decode-kernel instantiation, the mean of each counter over
its last ``--timed`` dispatches (a counter present in several files is read
from the last of them) and, where the counters are present, the LDS
bank-conflict share (``SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS``: stalled
cycles per LDS-active cycle), ROCm's ``LDSBankConflict`` (``100 *
SQ_LDS_BANK_CONFLICT / GRBM_GUI_ACTIVE / CUs``, percent of GPU time per CU,
with ``GRBM_GUI_ACTIVE`` per XCD: rocprofv3 writes it summed over the XCDs) and
the wait share (``SQ_WAIT_ANY / SQ_WAVE_CYCLES``: wave time spent waiting,
barriers and memory included).
"""

from __future__ import annotations

import argparse
import csv
import json

COPY_BYTES = 1 << 30
KERNEL = "decode_kernel"


def _read(path: str):
    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    decode, copies = [], []
    for r in rows:
        v = float(r["Counter_Value"])
        if KERNEL in r["Kernel_Name"]:
            decode.append(v)
        elif "copyBuffer" in r["Kernel_Name"] and v * 1024 > COPY_BYTES / 4:
            copies.append(v)
    if not copies:
        raise ValueError(f"{path}: no calibration copy found (run bench.py with --copy-calibration)")
    return decode, copies


def traffic(fetch_csv: str, write_csv: str, timed: int) -> dict:
    out = {}
    for name, path in (("fetch", fetch_csv), ("write", write_csv)):
        decode, copies = _read(path)
        if len(decode) < timed:
            raise ValueError(f"{path}: {len(decode)} decode dispatches, fewer than {timed}")
        copy_kib = sum(copies) / len(copies)
        scale = COPY_BYTES / (copy_kib * 1024)
        kib = sum(decode[-timed:]) / timed
        out[name] = {"kib_per_dispatch": round(kib, 1), "copy_kib": round(copy_kib, 1), "scale": round(scale, 5),
                     "bytes": int(round(kib * 1024 * scale))}
    out["total_bytes"] = out["fetch"]["bytes"] + out["write"]["bytes"]
    return out


def sq_summary(paths, timed: int, cus: int = 256, xcds: int = 8) -> dict:
    """Per decode-kernel instantiation: mean of each counter over its last `timed` dispatches."""
    per = {}  # kernel -> counter -> [values in dispatch order]
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"]
                if KERNEL not in name:
                    continue
                k = name[name.index(KERNEL):].split("(")[0]
                per.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    out = {}
    for k, cs in per.items():
        m = {c: sum(v[-timed:]) / len(v[-timed:]) for c, v in cs.items()}
        d = {"dispatches": min(len(v) for v in cs.values()), "mean": {c: round(x, 1) for c, x in m.items()}}
        if "SQ_LDS_BANK_CONFLICT" in m and m.get("SQ_ACTIVE_INST_LDS"):
            d["lds_bank_conflict_per_active_cycle"] = round(m["SQ_LDS_BANK_CONFLICT"] / m["SQ_ACTIVE_INST_LDS"], 5)
        if "SQ_LDS_BANK_CONFLICT" in m and m.get("GRBM_GUI_ACTIVE"):
            d["LDSBankConflict_pct"] = round(100 * m["SQ_LDS_BANK_CONFLICT"] / (m["GRBM_GUI_ACTIVE"] / xcds) / cus, 4)
        if "SQ_WAIT_ANY" in m and m.get("SQ_WAVE_CYCLES"):
            d["wait_share"] = round(m["SQ_WAIT_ANY"] / m["SQ_WAVE_CYCLES"], 4)
        out[k] = d
    return out


def main():
    import sys

    if len(sys.argv) > 1 and sys.argv[1] == "sq":
        ap = argparse.ArgumentParser(prog="counters sq")
        ap.add_argument("csv", nargs="+")
        ap.add_argument("--timed", type=int, default=256)
        a = ap.parse_args(sys.argv[2:])
        print(json.dumps(sq_summary(a.csv, a.timed), indent=1))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("fetch_csv")
    ap.add_argument("write_csv")
    ap.add_argument("--timed", type=int, default=1024)
    a = ap.parse_args()
    print(json.dumps(traffic(a.fetch_csv, a.write_csv, a.timed), indent=1))


if __name__ == "__main__":
    main()
