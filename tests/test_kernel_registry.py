"""KernelRegistry (reference src/runtime/KernelRegistry.mm:22-103) on the
host: admitted.json artifacts are taken only when their contract equals the
current device's contract text, under decoder_* directories, with a
candidate that names the contract's function; everything else leaves the
region on its template kernel.  The usage audit counts completed calls."""
import json

import pytest


def _artifact(contract, function="add_rmsnorm", source="add_rmsnorm?threads=256", wg=256,
              status="admitted", version=1):
    return ('{"version":%d,"status":"%s","contract":%s,"candidate":{"function_name":"%s",'
            '"source":"%s","workgroup_size":%d}}' % (version, status, contract, function, source,
                                                     wg))


def test_registry_takes_only_matching_artifacts(host, tmp_path):
    rt = host.HipRuntime()  # no device needed: the contract text is host data
    add = host.kernel_contract_text(rt, "AddRMSNorm")
    norm = host.kernel_contract_text(rt, "decoder_rmsnorm")
    assert json.loads(add)["pattern"] == "decoder_residual_rmsnorm"
    assert json.loads(add)["target"]["arch"] == "gfx950"
    lib = tmp_path / "lib"
    (lib / "decoder_residual_rmsnorm").mkdir(parents=True)
    (lib / "decoder_residual_rmsnorm" / "admitted.json").write_text(_artifact(add))
    # another device's contract
    other = json.loads(norm)
    other["target"]["device"] = "some other GPU"
    (lib / "decoder_rmsnorm").mkdir()
    (lib / "decoder_rmsnorm" / "admitted.json").write_text(
        _artifact(json.dumps(other, separators=(",", ":")), "rmsnorm", "rmsnorm?threads=128", 128))
    # wrong function, bad JSON, no artifact, not a decoder_ directory
    (lib / "decoder_silu_mul").mkdir()
    (lib / "decoder_silu_mul" / "admitted.json").write_text(
        _artifact(host.kernel_contract_text(rt, "SiLUMul"), "rmsnorm", "rmsnorm?threads=64", 64))
    (lib / "decoder_unknown").mkdir()
    (lib / "decoder_unknown" / "admitted.json").write_text("{not json")
    (lib / "decoder_empty").mkdir()
    (lib / "notes").mkdir()
    (lib / "notes" / "admitted.json").write_text(_artifact(add))
    reg = host.KernelRegistry()
    log = reg.load(rt, str(lib))
    assert reg.size() == 1, log
    entry = reg.find("decoder_residual_rmsnorm")
    assert entry == {"function_name": "add_rmsnorm", "source": "add_rmsnorm?threads=256",
                     "workgroup_size": 256}
    assert reg.find("decoder_rmsnorm") is None and "another contract or device" in log
    assert "decoder_silu_mul: invalid candidate" in log
    assert "decoder_empty: no admitted.json" in log
    assert "notes" not in log
    assert "template kernels" in host.KernelRegistry().load(rt, "")
    # a retry or another version is not an admitted artifact
    (lib / "decoder_residual_rmsnorm" / "admitted.json").write_text(_artifact(add, status="retry"))
    assert host.KernelRegistry().load(rt, str(lib)).count("loaded") == 0


def test_registry_usage_audit(host):
    reg = host.KernelRegistry()
    a = reg.track("bucket 1 residual norms", "decoder_residual_rmsnorm", "generated",
                  "add_rmsnorm?threads=256", 64)
    b = reg.track("bucket 1 input norm", "decoder_rmsnorm", "template", "rmsnorm?", 1)
    reg.completed([a, b])
    reg.completed([a])
    text = reg.report()
    assert "2 calls, 128 dispatches" in text and "1 calls, 1 dispatches" in text
    assert "dispatches: generated 128, template 1" in text
    reg.reset_usage()
    assert "dispatches: generated 0, template 0" in reg.report()
    with pytest.raises(Exception):
        reg.completed([5])
