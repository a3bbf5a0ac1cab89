"""The committed HBM-traffic measurement is reported only for the kernel sources it was made
from (cortexsdr_amd/traffic.py): a record whose source digest differs from the tree's reads
as stale, so bench.py cannot label an older kernel's traffic as the current one's."""
import json
import os

from cortexsdr_amd import traffic

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_committed_record_names_its_sources():
    path = os.path.join(ROOT, "profiles", "hsdb_gather_cfg2_traffic.json")
    with open(path) as f:
        t = json.load(f)
    assert t["sources"] == list(traffic.HSDB_SOURCES)
    assert len(t["source_digest"]) == 16
    assert t["traffic_bytes"] > t["algorithmic_bytes"] * 0.9


def test_stale_record_is_refused(tmp_path):
    rec = {"traffic_bytes": 123, "sources": list(traffic.HSDB_SOURCES),
           "source_digest": traffic.source_digest()}
    p = tmp_path / "t.json"
    p.write_text(json.dumps(rec))
    got, why = traffic.load_current(str(p))
    assert got is not None and why is None
    rec["source_digest"] = "0" * 16
    p.write_text(json.dumps(rec))
    got, why = traffic.load_current(str(p))
    assert got is None and why.startswith("stale")
    got, why = traffic.load_current(str(tmp_path / "missing.json"))
    assert got is None and why == "missing"


def test_measure_scales_by_the_calibration_copy(tmp_path):
    head = ("Dispatch_Id,Kernel_Name,Grid_Size,Counter_Name,Counter_Value\n")
    f = tmp_path / "f.csv"
    w = tmp_path / "w.csv"
    f.write_text(head + "1,__amd_rocclr_copyBuffer,131072,FETCH_SIZE,131072\n"
                 "2,void gatherw_kernel<8>,1,FETCH_SIZE,1000\n"
                 "3,void gatherw_kernel<8>,1,FETCH_SIZE,1002\n")
    w.write_text(head + "1,__amd_rocclr_copyBuffer,131072,WRITE_SIZE,262144\n"
                 "2,void gatherw_kernel<8>,1,WRITE_SIZE,10\n")
    m = traffic.measure(str(f), str(w), "gatherw_kernel")
    # fetch reads half the copied KiB: factor 0.5; write factor 1
    assert m["calibration"]["fetch_scale"] == 0.5
    assert m["traffic_bytes"] == int((1001 / 0.5 + 10) * 1024)
