"""Table of the LDS swizzle probe: per pattern, SQ_LDS_BANK_CONFLICT and SQ_LDS_IDX_ACTIVE
cycles per LDS instruction (dispatches in launch order, names from the probe's output).

usage: python lds_swizzle_report.py <probe stdout> <rocprofv3 pmc_counter_collection.csv>
"""

import collections
import csv
import sys


def main(log_path: str, csv_path: str) -> None:
    names = [line.split(" ", 2)[2].strip() for line in open(log_path) if line.startswith("pattern ")]
    counters = collections.defaultdict(dict)
    for row in csv.DictReader(open(csv_path)):
        if "probe_" in row["Kernel_Name"]:
            counters[int(row["Dispatch_Id"])][row["Counter_Name"]] = float(row["Counter_Value"])
    ids = sorted(counters)
    if len(ids) != len(names):
        raise SystemExit(f"{len(ids)} dispatches but {len(names)} pattern names")
    print(f"{'pattern':62s} {'conflict cyc/inst':>18s} {'LDS cyc/inst':>13s}")
    for i, name in zip(ids, names):
        c = counters[i]
        n = c["SQ_INSTS_LDS"]
        print(f"{name:62s} {c['SQ_LDS_BANK_CONFLICT'] / n:18.2f} {c['SQ_LDS_IDX_ACTIVE'] / n:13.2f}")


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
