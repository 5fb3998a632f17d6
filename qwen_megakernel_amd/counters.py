"""HBM traffic per decode launch from rocprofv3 counter CSVs.

Usage (after two counter runs of ``bench.py --copy-calibration``, one with
``--pmc FETCH_SIZE`` and one with ``--pmc WRITE_SIZE``, both ``-f csv``):

    python -m qwen_megakernel_amd.counters FETCH.csv WRITE.csv --timed 1024

``FETCH_SIZE`` / ``WRITE_SIZE`` are in KiB per dispatch.  Each counter is
scaled by the ratio of the known size of the calibration copy (1 GiB read and
1 GiB written) to what the same counter reads for that copy, then averaged
over the last ``--timed`` decode dispatches (the timed region of the run).
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("fetch_csv")
    ap.add_argument("write_csv")
    ap.add_argument("--timed", type=int, default=1024)
    a = ap.parse_args()
    print(json.dumps(traffic(a.fetch_csv, a.write_csv, a.timed), indent=1))


if __name__ == "__main__":
    main()
