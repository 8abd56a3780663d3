"""bench.py's live HBM-traffic measurement parses rocprofv3's counter CSV and scales each counter
by its reading of the 256 MiB copy; without rocprofv3 (this container) it falls back to the
committed PMC summary and says so.  No GPU is touched."""
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

HEADER = ('"Correlation_Id","Dispatch_Id","Agent_Id","Queue_Id","Process_Id","Thread_Id","Grid_Size",'
          '"Kernel_Id","Kernel_Name","Workgroup_Size","LDS_Block_Size","Scratch_Size","VGPR_Count",'
          '"Accum_VGPR_Count","SGPR_Count","Counter_Name","Counter_Value","Start_Timestamp","End_Timestamp"')


def _row(i, name, counter, value):
    return f'{i},{i},"Agent 1",1,1,1,256,7,"{name}",256,0,0,4,0,16,"{counter}",{value},1,2'


def test_live_pass_parses_the_counter_csv(monkeypatch, tmp_path):
    fake_tool = tmp_path / "rocprofv3"
    fake_tool.write_text("#!/bin/sh\n")
    fake_tool.chmod(0o755)
    monkeypatch.setattr("shutil.which", lambda name: str(fake_tool))
    readings = {"FETCH_SIZE": (512085.5, 131072.0), "WRITE_SIZE": (256.0, 262144.0)}

    def fake_run(cmd, **kwargs):
        counter = cmd[cmd.index("--pmc") + 1]
        out = pathlib.Path(cmd[cmd.index("-d") + 1]) / "host" / f"{counter.lower()}_counter_collection.csv"
        out.parent.mkdir(parents=True)
        dom, copy = readings[counter]
        rows = [HEADER, _row(1, "void at::native::fill", counter, 3.0)]
        for i in range(3):
            rows.append(_row(2 + 2 * i, "logsumexp_serial_bf16_v256u8w4", counter, dom))
            rows.append(_row(3 + 2 * i, "__amd_rocclr_copyBuffer", counter, copy))
        out.write_text("\n".join(rows) + "\n")
        return subprocess.CompletedProcess(cmd, 0)

    monkeypatch.setattr("subprocess.run", fake_run)
    for k in [k for k in bench.os.environ if k.startswith("ROCPROF")]:
        monkeypatch.delenv(k)
    monkeypatch.setenv("LD_PRELOAD", "")
    traffic, info = bench.pmc_traffic(live=True)
    fetch_scale, write_scale = 262144 / 131072.0, 262144 / 262144.0
    assert traffic == round((512085.5 * fetch_scale + 256.0 * write_scale) * 1024)
    assert info["source"].startswith("rocprofv3") and info["fetch_scale"] == 2.0


def test_falls_back_to_the_committed_summary(monkeypatch):
    monkeypatch.setattr("shutil.which", lambda name: None)
    traffic, info = bench.pmc_traffic(live=True)
    assert info["source"] == "profiles/logsumexp_bf16_16384x32000_pmc.md"
    assert traffic is not None and traffic > 1_048_608_768


def test_cfg5_annotation_names_the_selected_kernel_and_its_profile():
    """The cfg5 entry names the head-dim-128 kernel attention.use_w64 picks at its shape, and
    its MFMA figures come from that kernel's committed counter summary."""
    from neptune_codegen import attention as A

    assert bench.kernel_of(True).startswith(
        "64 queries" if A.use_w64(128, True, 4096, 4096) else "32 queries")
    assert bench.kernel_of(False).startswith("64 queries")
    pmc = bench.attention_pmc()
    assert pmc is not None and 0.3 < pmc["mfma_busy_frac"] < 0.8 and 1.0 < pmc["clock_ghz_first_call"] < 2.5
