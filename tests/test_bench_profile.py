"""bench.py's link to the committed rocprofv3 summaries: the HBM traffic of the
headline GEMV is read from profiles/gemv_q4_0_14336x4096_pmc.txt, and the M=512
GEMM's MFMA busy fraction from profiles/gemm_q4_0_14336x4096_m512_mfma_pmc.txt,
only when the summary's kernel_sources_sha256 names the sources of this tree."""
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


def _write_mfma(tmp_path, digest, line="MFMA utilisation = A / B = 35.6% (all 256 CUs hold work)."):
    p = tmp_path / "mfma.txt"
    p.write_text("# summary\n"
                 f"kernel_sources_sha256: {digest}   (python bench.py --sources-digest gemm)\n"
                 f"{line}\n")
    return p


def test_mfma_busy_from_current_summary(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "GEMM_PMC_PROFILE", _write_mfma(tmp_path, bench.kernel_sources_digest("gemm")))
    frac, status = bench.mfma_busy_from_profile()
    assert status == "current" and abs(frac - 0.356) < 1e-12


def test_mfma_busy_stale_or_missing(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "GEMM_PMC_PROFILE", _write_mfma(tmp_path, "0123456789abcdef"))
    assert bench.mfma_busy_from_profile() == (None, "stale")
    monkeypatch.setattr(bench, "GEMM_PMC_PROFILE", _write_mfma(tmp_path, bench.kernel_sources_digest("gemm"),
                                                                line="no figure here"))
    assert bench.mfma_busy_from_profile() == (None, "missing")


def test_committed_gemm_counters_give_a_busy_fraction():
    frac, status = bench.mfma_busy_from_profile()
    assert status == "current" and 0.2 < frac < 1.0


def test_digest_covers_every_gemv_source():
    assert len(bench.kernel_sources_digest()) == 16
    assert all((bench.ROOT / rel).is_file() for rel in bench.GEMV_KERNEL_SOURCES)


def _stamp(text: str, key: str) -> list[str]:
    return [ln.split()[1] for ln in text.splitlines() if ln.startswith(key + ":") and len(ln.split()) > 1]


def test_committed_headline_summaries_are_current():
    """The committed kernel-trace and counter summaries of the headline GEMV
    were taken from this tree's GEMV sources: a change to them without a new
    profile fails here, before the bench line reports traffic as stale."""
    want = bench.kernel_sources_digest()
    for name in ("gemv_q4_0_14336x4096_pmc.txt", "gemv_q4_0_14336x4096_kernel_trace.txt"):
        text = (bench.ROOT / "profiles" / name).read_text()
        assert _stamp(text, "kernel_sources_sha256") == [want], (name, _stamp(text, "kernel_sources_sha256"), want)
    assert bench.traffic_from_profile()[1] == "current"


def test_every_committed_summary_is_current():
    """Every summary under profiles/ names the kernel group it profiles and the
    digest of that group's sources (python bench.py --sources-digest GROUP); it
    must equal the digest of this tree's sources, so that no committed figure
    describes kernels that have since changed."""
    files = sorted((bench.ROOT / "profiles").glob("*.txt"))
    assert len(files) >= 10
    for f in files:
        text = f.read_text()
        groups = _stamp(text, "kernel_group")
        assert len(groups) == 1 and groups[0] in bench.KERNEL_SOURCE_GROUPS, (f.name, groups)
        want = bench.kernel_sources_digest(groups[0])
        assert _stamp(text, "kernel_sources_sha256") == [want], (f.name, groups[0], want)


def test_source_groups_name_existing_files():
    for group, paths in bench.KERNEL_SOURCE_GROUPS.items():
        assert paths and all((bench.ROOT / rel).is_file() for rel in paths), group
    # every kernel translation unit belongs to some group
    hip = {p.relative_to(bench.ROOT).as_posix() for p in (bench.ROOT / "woolly_amd" / "csrc").glob("*.hip")}
    covered = set(sum(bench.KERNEL_SOURCE_GROUPS.values(), ()))
    assert hip - covered <= {"woolly_amd/csrc/api.hip", "woolly_amd/csrc/gguf.hip", "woolly_amd/csrc/dequant.hip",
                             "woolly_amd/csrc/probe.hip"}, hip - covered
