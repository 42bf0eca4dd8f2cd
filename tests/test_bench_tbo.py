"""bench.py --tbo-sql: the test-backend-ops perf rows the reference's analysis scripts read.

The checks restate what those scripts require, without running them: bench/analyze.py:42-56 keeps only the
CREATE TABLE / INSERT statements of a file, loads them into SQLite and selects (op_name, op_params, supported,
time_us) where test_mode = 'perf', splitting op_params with the regex below; bin/mm-gbps.py:24-46 accepts a
MUL_MAT case only with an f32, unbatched, contiguous right-hand side and computes its bytes as
m*k/elements*bytes + n*k*4 + m*n*4.
"""
import re
import sqlite3

import bench

EXTRA = {
    "matvec_sweep_op_us": {"q4_0 4096x14336 n=1": {"us": 11.25, "gbs": 2944.3},
                           "q8_0 1024x4096 n=8": {"us": 6.5, "gbs": 700.0}},
    "fa_decode": {"by_ctx": {"8192": {"us": 12.47, "bytes": 33587200}}},
    "fa_decode_q4_0_kv": {"by_ctx": {"2048": {"us": 8.04, "bytes": 2392064}}},
    "kquant": {"q6_K 128256x4096 n=1": {"kernel": {"us": 95.2}, "op": {"us": 97.3, "gbs": 4434.3}},
               "q6_K 128256x4096 n=8": {"kernel": {"us": 134.8}}},
}


def test_tbo_sql_reads_like_test_backend_ops(tmp_path):
    path = tmp_path / "bench.sql"
    bench.write_tbo_sql(str(path), EXTRA, "AMD Instinct MI355X")
    text = path.read_text()
    stmts = re.findall(r"(CREATE TABLE.*?\);|INSERT INTO.*?\);)\s*$", text, re.S | re.M)
    assert len(stmts) == 1 + 5  # the kernel-only K-quant entry is not a test-backend-ops row
    db = sqlite3.connect(":memory:")
    db.executescript("\n".join(stmts))
    rows = db.execute("SELECT op_name, op_params, supported, time_us, bandwidth_gb_s FROM test_backend_ops "
                      "WHERE test_mode='perf'").fetchall()
    assert len(rows) == 5
    mm = {}
    for op, params, supported, us, gbs in rows:
        kv = dict(re.findall(r"(\w+)=(\[[^\]]*\]|[^,]+)", params))
        assert supported == 1 and us > 0
        if op == "MUL_MAT":
            assert kv["type_b"] == "f32" and kv["bs"] == "[1,1]" and kv["nr"] == "[1,1]"
            assert kv["per"] == "[0,1,2,3]" and kv["o"] == "1"
            assert all(kv[f] == "0" for f in ("k_v", "src_overlap", "m_v", "pad"))
            mm[(kv["type_a"], int(kv["m"]), int(kv["k"]), int(kv["n"]))] = (us, gbs)
        else:
            assert op == "FLASH_ATTN_EXT" and kv["hsk"] == "128" and kv["type_K"] in ("f16", "q4_0")
    us, gbs = mm[("q4_0", 4096, 14336, 1)]
    nbytes = 4096 * 14336 // 32 * 18 + 14336 * 4 + 4096 * 4
    assert abs(gbs - nbytes / (us * 1e-6) / 1e9) < 1e-3
    assert ("q8_0", 1024, 4096, 8) in mm
    us, gbs = mm[("q6_K", 128256, 4096, 1)]
    assert us == 97.3 and abs(gbs - (128256 * 4096 // 256 * 210 + 4096 * 4 + 128256 * 4) / 97.3e-6 / 1e9) < 1e-3
