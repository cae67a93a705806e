"""Hip artifacts on the CPU: what the reader refuses before a device is involved
(crates/modelspec-core/src/artifact.rs:1-35, 330-420: E-ARTIFACT-001 for a missing manifest, an
unknown format version or backend, a manifest that is not JSON)."""
import json
import os

import pytest

from modelspec_amd import api


def refused(path):
    with pytest.raises(api.MsxError) as e:
        api.check_artifact(path)
    return e.value


def test_a_directory_without_a_manifest_is_refused(tmp_path):
    e = refused(tmp_path)
    assert e.code == -7 and "E-ARTIFACT-001" in str(e)


@pytest.mark.parametrize("text", ["not json", json.dumps({"format_version": 2, "backend": "Hip"}),
                                  json.dumps({"format_version": 1, "backend": "Vulkan"}),
                                  json.dumps({"format_version": 1, "backend": "Hip"})])
def test_a_manifest_of_another_version_backend_or_form_is_refused(tmp_path, text):
    open(os.path.join(tmp_path, "artifact.json"), "w").write(text)
    e = refused(tmp_path)
    assert e.code == -7 and "E-ARTIFACT-001" in str(e)
