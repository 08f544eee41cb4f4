"""CPU tests of deployment loading (custom_ops_amd/loader.py): offline build with
a metadata sidecar, validated precompiled load, strict (no-compile) policy and
fail-closed dispatcher ownership. They follow the intent of the reference's
tests/test_custom_ops_loading.py (fresh processes for every dispatcher state,
rejection before the library is opened, copies and untracked registrations
refused), for this build's ctypes-loaded C-ABI library.
"""
import json
import os
import shutil
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_py(code: str, timeout: int = 300):
    """Run `code` in a fresh interpreter (fresh dispatcher) from the repo root."""
    env = dict(os.environ, PYTHONPATH=ROOT)
    env.pop("MI355_FA_LIB", None)
    res = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], cwd=ROOT, env=env,
                         capture_output=True, text=True, timeout=timeout)
    return res.returncode, res.stdout, res.stderr


@pytest.fixture(scope="module")
def exported(tmp_path_factory):
    """One offline build shared by the tests (hipcc cross-compiles, no GPU)."""
    from custom_ops_amd.loader import FAOps
    out = tmp_path_factory.mktemp("export")
    lib = FAOps().build(out)
    return lib


def copy_pair(lib, dst_dir):
    dst_dir.mkdir(parents=True, exist_ok=True)
    dst = dst_dir / lib.name
    shutil.copy2(lib, dst)
    shutil.copy2(str(lib) + ".json", str(dst) + ".json")
    return dst


def test_build_exports_library_and_sealed_sidecar_without_loading(exported):
    from custom_ops_amd import _lib
    from custom_ops_amd.loader import ARTIFACT_FORMAT, _digest_file, seal_of
    md = json.loads(open(str(exported) + ".json").read())
    assert md["format"] == ARTIFACT_FORMAT
    assert md["contract"]["namespace"] == "recsys_ops"
    assert md["targets"] == ["gfx950"]
    assert md["contract"]["schemas"] == {
        "recsys_ops::mha_fwd_with_mask":
        "recsys_ops::mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor"}
    assert md["contract"]["meta_ops"] == ["mha_fwd_with_mask"]
    assert md["contract"]["abi"] == _lib.ABI_VERSION
    assert md["payload"] == {"file": exported.name, "bytes": exported.stat().st_size,
                             "sha256": _digest_file(exported)}
    assert "-packed-fp32-ops" in md["provenance"]["flags"]
    assert len(md["provenance"]["sources_sha256"]) == 64
    assert md["seal"] == seal_of(md)
    # the in-process library is untouched: building never loads
    assert _lib.loaded_path() is None or "export" not in _lib.loaded_path()


def test_precompiled_load_in_fresh_process_is_strict(exported):
    rc, out, err = run_py(f"""
        import torch
        from custom_ops_amd import ops, CustomOpsError
        ops.load_precompiled("fa", {str(exported)!r})
        assert not ops.allow_jit
        assert ops.groups == {{"fa": "loaded"}}, ops.groups
        s = str(torch.ops.recsys_ops.mha_fwd_with_mask.default._schema)
        assert s.startswith("recsys_ops::mha_fwd_with_mask(Tensor q"), s
        assert torch._C._dispatch_has_kernel_for_dispatch_key(
            "recsys_ops::mha_fwd_with_mask", "Meta")
        from custom_ops_amd import _lib
        import os
        assert _lib.loaded_path() == os.path.realpath({str(exported)!r})
        # the same file again is idempotent
        ops.load_precompiled("fa", {str(exported)!r})
        print("OK")
    """)
    assert rc == 0 and "OK" in out, err[-3000:]


def test_strict_facade_never_compiles_or_opens_the_dev_library():
    rc, out, err = run_py("""
        from custom_ops_amd import ops, CustomOpsError
        from custom_ops_amd import build, _lib
        called = []
        build.build = lambda *a, **k: called.append(1)
        ops.disable_jit()
        try:
            ops.ensure_loaded("fa")
        except CustomOpsError as e:
            assert "load_precompiled" in str(e), e
        else:
            raise SystemExit("strict ensure_loaded did not raise")
        assert ops.is_available("fa") is False
        assert not called and _lib.loaded_path() is None
        print("OK")
    """)
    assert rc == 0 and "OK" in out, err[-3000:]


@pytest.mark.parametrize("path,value,msg", [
    (("contract", "namespace"), "other_ops", "seal is broken"),
    (("format",), "custom_ops_amd.artifact/1", "format mismatch"),
    (("contract", "group_version"), "2", "seal is broken"),
    (("targets",), ["gfx942", "gfx950"], "seal is broken"),
    (("payload", "bytes"), 1, "seal is broken"),
])
def test_edited_sidecar_rejected_before_open(exported, tmp_path, path, value, msg):
    """An edited sidecar (seal not recomputed) never gets as far as dlopen."""
    lib = copy_pair(exported, tmp_path / "m")
    side = str(lib) + ".json"
    md = json.loads(open(side).read())
    node = md
    for key in path[:-1]:
        node = node[key]
    node[path[-1]] = value
    open(side, "w").write(json.dumps(md))
    rc, out, err = run_py(f"""
        from custom_ops_amd.loader import FAOps, CustomOpsError
        from custom_ops_amd import _lib
        try:
            FAOps().load_precompiled({str(lib)!r})
        except CustomOpsError as e:
            print("ERR", e)
        assert _lib.loaded_path() is None      # rejected before dlopen
    """)
    assert rc == 0 and "ERR" in out and msg in out, (out, err[-2000:])


def test_resealed_mismatches_name_the_section(exported, tmp_path):
    """A consistently resealed but wrong sidecar fails on the section that differs."""
    from custom_ops_amd.loader import CustomOpsError, FAOps, seal_of
    for i, (mutate, msg) in enumerate([
        (lambda md: md["contract"]["schemas"].update(
            {"recsys_ops::mha_fwd_with_mask": "recsys_ops::mha_fwd_with_mask(Tensor q) -> Tensor"}),
         "contract mismatch (schemas"),
        (lambda md: md["contract"].update({"namespace": "other_ops"}), "contract mismatch (namespace"),
        (lambda md: md["contract"].update({"abi": 1}), "contract mismatch (abi"),
        (lambda md: md["runtime"].update({"torch": "1.13"}), "runtime mismatch (torch"),
        (lambda md: md.update({"targets": ["GFX950"]}), "invalid offload target"),
        (lambda md: md["payload"].update({"bytes": 1}), "payload size mismatch"),
    ]):
        lib = copy_pair(exported, tmp_path / f"case{i}")
        side = str(lib) + ".json"
        md = json.loads(open(side).read())
        mutate(md)
        md["seal"] = seal_of(md)
        open(side, "w").write(json.dumps(md))
        with pytest.raises(CustomOpsError, match=msg.replace("(", r"\(")):
            FAOps().load_precompiled(lib)


def test_visible_target_mismatch_rejected(exported, monkeypatch):
    from custom_ops_amd import loader
    monkeypatch.setattr(loader, "_visible_archs", lambda: {"gfx942"})
    with pytest.raises(loader.CustomOpsError, match="target mismatch"):
        loader.FAOps().load_precompiled(exported)


def test_modified_or_missing_files_rejected(exported, tmp_path):
    from custom_ops_amd.loader import FAOps, CustomOpsError
    lib = copy_pair(exported, tmp_path / "t")
    with open(lib, "r+b") as f:          # same size, one byte changed
        f.seek(4096)
        b = f.read(1)
        f.seek(4096)
        f.write(bytes([b[0] ^ 0xFF]))
    with pytest.raises(CustomOpsError, match="payload digest mismatch"):
        FAOps().load_precompiled(lib)
    lib2 = copy_pair(exported, tmp_path / "n")
    os.remove(str(lib2) + ".json")
    with pytest.raises(CustomOpsError, match="failed"):
        FAOps().load_precompiled(lib2)
    with pytest.raises(CustomOpsError):
        FAOps().load_precompiled(tmp_path / "absent.so")


def test_copy_of_loaded_library_is_a_dispatcher_conflict(exported, tmp_path):
    other = copy_pair(exported, tmp_path / "copy")
    rc, out, err = run_py(f"""
        from custom_ops_amd.loader import FAOps, CustomOpsError
        FAOps().load_precompiled({str(exported)!r})
        try:
            FAOps().load_precompiled({str(other)!r})
        except CustomOpsError as e:
            print("ERR", e)
    """)
    assert rc == 0 and "cannot serve it in this process" in out, (out, err[-2000:])


def test_untracked_registration_is_fail_closed(exported):
    rc, out, err = run_py(f"""
        import torch
        lib = torch.library.Library("recsys_ops", "FRAGMENT")
        lib.define("mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor")
        from custom_ops_amd.loader import FAOps, CustomOpsError
        from custom_ops_amd import _lib
        try:
            FAOps().load_precompiled({str(exported)!r})
        except CustomOpsError as e:
            print("ERR", e)
        assert _lib.loaded_path() is None
    """)
    assert rc == 0 and "untracked library" in out, (out, err[-2000:])


def test_build_refuses_to_overwrite_a_loaded_library(exported):
    rc, out, err = run_py(f"""
        from custom_ops_amd.loader import FAOps, CustomOpsError
        FAOps().load_precompiled({str(exported)!r})
        try:
            FAOps().build({str(exported.parent)!r})
        except CustomOpsError as e:
            print("ERR", e)
    """, timeout=600)
    assert rc == 0 and "cannot overwrite a library loaded" in out, (out, err[-2000:])


def test_policy_is_explicit_bool():
    from custom_ops_amd import RecsysOps
    from custom_ops_amd.loader import FAOps
    for obj in (RecsysOps(), FAOps()):
        with pytest.raises(TypeError):
            obj.configure(allow_jit="no")
        assert obj.disable_jit().allow_jit is False


def test_failure_after_open_is_sticky(exported):
    """A load that fails after the library was opened marks the operator broken:
    retrying in the same process is refused instead of half-registering twice."""
    rc, out, err = run_py(f"""
        from custom_ops_amd import fa
        from custom_ops_amd.loader import FAOps, CustomOpsError
        orig = fa.register
        def boom():
            raise RuntimeError("injected registration failure")
        fa.register = boom
        try:
            FAOps().load_precompiled({str(exported)!r})
        except CustomOpsError as e:
            print("ERR1", e)
        fa.register = orig
        try:
            FAOps().load_precompiled({str(exported)!r})
        except CustomOpsError as e:
            print("ERR2", e)
    """)
    assert rc == 0 and "injected registration failure" in out, (out, err[-2000:])
    assert "ERR2" in out and "failed midway" in out, (out, err[-2000:])
