"""The FIT-only trainer process (dp_model_train), the class_model_train drop-in.

Contract followed: native/class_model_train.cu:25-86 (plan check, output
directory, receipts, exit codes), native/class_model_dataset_contract.hpp:23-38
(dense descriptor) and native/class_native_training.cuh:16-33 (hyperparameters).
The plan and dataset checks run without a GPU; `fit` is a GPU test whose model
must equal, byte for byte, the model the in-process C API trains from the same
rows and parameters.
"""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

EXE = os.path.join(ROOT, "decision-programs_amd", "bin", "dp_model_train")
LIB = os.path.join(ROOT, "decision-programs_amd", "lib", "libdpgbdt_hip.so")


def sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def run(*args):
    p = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=300)
    return p.returncode, p.stdout, p.stderr


def manifest():
    rc, out, err = run("source-manifest")
    assert rc == 0, err
    return json.loads(out)


def write_dataset(tmp, rows=3000, features=10, stride=12, classes=3, seed=5, bad_label=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, stride)).astype(np.float32)
    x[:, features:] = 7.0  # padding columns beyond the declared features
    x[rng.random((rows, stride)) < 0.05] = np.nan
    y = (np.nan_to_num(x[:, 0]) * 2 + np.nan_to_num(x[:, 1]) > 0).astype(np.uint32)
    y = (y + (np.nan_to_num(x[:, 2]) > 0.5)) % classes
    if bad_label:
        y[17] = classes
    xp, yp = tmp / "values.f32", tmp / "labels.u32"
    x.tofile(xp)
    y.astype("<u4").tofile(yp)
    return x, y, {"format": "dense-fp32-u32-class-labels-1", "TEST_read": False,
                  "features": features, "classes": classes, "rows": rows, "row_stride": stride,
                  "FIT_rows": rows, "VALID_rows": 0, "preprocessing": "synthetic test rows",
                  "values_path": str(xp), "labels_path": str(yp),
                  "values_sha256": sha(xp), "labels_sha256": sha(yp)}


def write_plan(tmp, dataset, hp=None, **over):
    plan = {"format": "class-model-training-plan-1", "dataset": dataset,
            "hyperparameters": hp or {"rounds": 3, "max_depth": 3, "eta": 0.5, "max_bin": 64},
            "TEST_read": False, "VALID_read": False, "selection_performed": False,
            "training_performed": True, "native_library_path": LIB,
            "native_library_sha256": sha(LIB), "executable_sha256": sha(EXE),
            "source_manifest_sha256": manifest()["sha256"]}
    plan.update(over)
    path = tmp / "plan.json"
    path.write_text(json.dumps(plan))
    return path, sha(path)


def test_source_manifest_digests():
    m = manifest()
    for name, digest in m["files"].items():
        assert digest == sha(os.path.join(ROOT, "decision-programs_amd", "csrc", name))
    compact = json.dumps(m["files"], separators=(",", ":"))
    assert m["sha256"] == hashlib.sha256(compact.encode()).hexdigest()
    assert list(m["files"]) == sorted(m["files"])


def test_usage_is_an_error():
    rc, _, err = run()
    assert rc == 1 and "usage" in err


def test_check_plan_accepts(tmp_path):
    _, _, ds = write_dataset(tmp_path)
    plan, pin = write_plan(tmp_path, ds)
    rc, out, err = run("--check-plan", str(plan), pin)
    assert rc == 0, err
    o = json.loads(out)
    assert o["checked"] is True and o["CUDA_executed"] is False
    assert o["hyperparameters"]["rounds"] == 3 and o["hyperparameters"]["lambda"] == 1.0
    assert o["dataset"]["rows"] == 3000


@pytest.mark.parametrize("change,message", [
    ({"TEST_read": True}, "FIT-only training protocol"),
    ({"training_performed": False}, "FIT-only training protocol"),
    ({"format": "other"}, "FIT-only training protocol"),
    ({"executable_sha256": "0" * 64}, "training executable differs"),
    ({"native_library_sha256": "1" * 64}, "pinned native library differs"),
    ({"native_library_sha256": "ABC"}, "64 lowercase"),
    ({"native_library_path": "lib.so"}, "must be absolute"),
    ({"source_manifest_sha256": "2" * 64}, "training source manifest differs"),
    ({"hyperparameters": {"rounds": 2, "max_depth": 2, "booster": "x"}},
     "unsupported training hyperparameter"),
    ({"hyperparameters": {"rounds": 0, "max_depth": 2}}, "positive rounds"),
    ({"hyperparameters": {"rounds": 2, "max_depth": 2, "eta": 0}}, "range"),
])
def test_check_plan_refusals(tmp_path, change, message):
    _, _, ds = write_dataset(tmp_path, rows=100)
    plan, pin = write_plan(tmp_path, ds, **change)
    rc, _, err = run("--check-plan", str(plan), pin)
    assert rc == 1 and message in err, err


@pytest.mark.parametrize("change,message", [
    ({"VALID_rows": 1}, "dense row/split range"),
    ({"FIT_rows": 99, "VALID_rows": 1}, "dense FIT-only or evaluation boundary"),
    ({"row_stride": 5}, "dense row/split range"),
    ({"classes": 1}, "dense feature/class range"),
    ({"classes": 2 ** 25}, "exact native FP32 label capacity"),
    ({"features": -1}, "dense features must be unsigned integer"),
    ({"values_sha256": "X" * 64}, "lowercase SHA256"),
    ({"values_path": "values.f32"}, "absolute dataset"),
    ({"preprocessing": ""}, "dense preprocessing identity"),
    ({"format": "idx"}, "dense format"),
])
def test_dense_descriptor_refusals(tmp_path, change, message):
    _, _, ds = write_dataset(tmp_path, rows=100)
    ds.update(change)
    plan, pin = write_plan(tmp_path, ds)
    rc, _, err = run("--check-plan", str(plan), pin)
    assert rc == 1 and message in err, err


def test_plan_pin_and_existing_output(tmp_path):
    _, _, ds = write_dataset(tmp_path, rows=100)
    plan, pin = write_plan(tmp_path, ds)
    rc, _, err = run("--check-plan", str(plan), "f" * 64)
    assert rc == 1 and "training plan SHA differs" in err
    out = tmp_path / "out"
    out.mkdir()
    rc, _, err = run("fit", str(plan), pin, str(out))
    assert rc == 1 and "output already exists" in err
    assert not (out / "failure.json").exists()  # the directory was not created by this run


@pytest.mark.gpu
@pytest.mark.parametrize("sampling", [{}, {"subsample": 0.8, "colsample_bynode": 0.5,
                                           "colsample_bytree": 0.9, "seed": 12}])
def test_fit_matches_in_process_training(tmp_path, dp, device, sampling):
    """dp_model_train fit writes the model the in-process API trains, also with the plan's
    row and column sampling keys (which the reference forwards to the library)."""
    import torch

    x, y, ds = write_dataset(tmp_path)
    hp = {"rounds": 4, "max_depth": 4, "eta": 0.5, "max_bin": 64, "lambda": 2, "alpha": 0.25,
          "min_child_weight": 0.5, **sampling}
    plan, pin = write_plan(tmp_path, ds, hp)
    out = tmp_path / "run"
    print(f"[cli] fit {ds['rows']} x {ds['features']} K={ds['classes']}", flush=True)
    rc, stdout, err = run("fit", str(plan), pin, str(out))
    assert rc == 0, err
    result = json.loads(stdout)
    for name in ("plan.json", "source-manifest.json", "model.json", "configuration.json",
                 "result.json", "result-seal.json"):
        assert (out / name).exists(), name
    seal = json.loads((out / "result-seal.json").read_text())
    assert seal["result_sha256"] == sha(out / "result.json")
    assert seal["model_sha256"] == sha(out / "model.json") == result["model_sha256"]
    assert result["plan_sha256"] == pin and result["FIT_rows"] == 3000
    assert json.loads((out / "plan.json").read_text()) == json.loads(plan.read_text())
    # the same fit through the in-process API
    values = torch.as_tensor(np.ascontiguousarray(x[:, :10]), device=device)
    labels = torch.as_tensor(y.astype(np.float32), device=device)
    dtrain = dp.DMatrix(values, labels)
    params = {"objective": "multi:softmax", "num_class": 3, "tree_method": "hist",
              "device": "cuda:0", "max_bin": 64, "max_depth": 4, "eta": 0.5, "lambda": 2,
              "alpha": 0.25, "gamma": 0, "min_child_weight": 0.5, "base_score": "[0,0,0]",
              "boost_from_average": 0, "seed": 0, **sampling}
    bst = dp.Booster(params, [dtrain])
    for r in range(4):
        bst.update(dtrain, r)
    assert bst.save_raw() == (out / "model.json").read_text()


@pytest.mark.gpu
def test_fit_failure_receipt(tmp_path, dp, device):
    _, _, ds = write_dataset(tmp_path, rows=500, bad_label=True)
    plan, pin = write_plan(tmp_path, ds)
    out = tmp_path / "run"
    print("[cli] fit with an out-of-range label", flush=True)
    rc, _, err = run("fit", str(plan), pin, str(out))
    assert rc == 1 and "exact native class IDs" in err
    failure = json.loads((out / "failure.json").read_text())
    assert failure["complete"] is False and failure["model_may_be_prepared"] is False
