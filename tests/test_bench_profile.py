"""bench.py's link to the committed rocprofv3 summaries: the HBM traffic of the
headline GEMV is read from profiles/gemv_q4_0_14336x4096_pmc.txt only when that
summary's kernel_sources_sha256 names the GEMV sources of this tree."""
import bench


def _write(tmp_path, digest, traffic="33299849"):
    p = tmp_path / "pmc.txt"
    p.write_text("# summary\n"
                 f"kernel_sources_sha256: {digest}   (python bench.py --sources-digest)\n"
                 f"traffic_bytes_per_launch: {traffic}\n")
    return p


def test_current_summary_gives_traffic(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "PMC_PROFILE", _write(tmp_path, bench.kernel_sources_digest()))
    assert bench.traffic_from_profile() == (33299849, "current")


def test_stale_summary_gives_none(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "PMC_PROFILE", _write(tmp_path, "0123456789abcdef"))
    assert bench.traffic_from_profile() == (None, "stale")


def test_missing_summary(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "PMC_PROFILE", tmp_path / "absent.txt")
    assert bench.traffic_from_profile() == (None, "missing")


def test_digest_covers_every_gemv_source():
    assert len(bench.kernel_sources_digest()) == 16
    assert all((bench.ROOT / rel).is_file() for rel in bench.GEMV_KERNEL_SOURCES)


def test_committed_headline_summaries_are_current():
    """The committed kernel-trace and counter summaries of the headline GEMV
    were taken from this tree's GEMV sources: a change to them without a new
    profile fails here, before the bench line reports traffic as stale."""
    want = bench.kernel_sources_digest()
    for name in ("gemv_q4_0_14336x4096_pmc.txt", "gemv_q4_0_14336x4096_kernel_trace.txt"):
        text = (bench.ROOT / "profiles" / name).read_text()
        recorded = [ln.split()[1] for ln in text.splitlines() if ln.startswith("kernel_sources_sha256:")]
        assert recorded == [want], (name, recorded, want)
    assert bench.traffic_from_profile()[1] == "current"
