"""The HTTP front of the text loop (src/main.rs:65-87, 138-155): the
/api/predict route, fix_encoding (utils/string.rs:3-7), and on the GPU the
route around the device text path with the reference vocabulary's ids."""
from __future__ import annotations

import html

import pytest

from rustcrates_amd import server


def test_fix_encoding_reads_utf8_bytes_as_windows_1252():
    # encoding_rs's WINDOWS_1252: every byte maps; the five cp1252 gaps are C1 controls
    assert server.fix_encoding("plain ascii") == "plain ascii"
    assert server.fix_encoding("é") == "Ã©"          # C3 A9
    assert server.fix_encoding("€") == "â‚¬"    # E2 82 AC
    assert server.fix_encoding("Á") == "Ã\u0081"          # C3 81: a gap byte
    assert server.fix_encoding("Ý") == "Ã\u009d"          # C3 9D: a gap byte


def test_predict_route_runs_predict_by_text_on_the_fixed_prompt():
    from fastapi.testclient import TestClient

    seen = []

    def fake(inputs):
        seen.append(inputs)
        return ["<bos> " + inputs[0] + " continued"]

    client = TestClient(server.create_app(fake))
    r = client.post("/api/predict", data={"prompt": "café & co"})
    assert r.status_code == 200 and r.headers["content-type"].startswith("text/html")
    assert seen == [["cafÃ© & co"]]
    assert html.escape(str(["<bos> cafÃ© & co continued"])) in r.text
    assert html.escape("café & co") in r.text  # the page keeps the prompt as typed
    assert client.post("/api/predict", data={}).status_code == 400
    assert client.get("/").status_code == 200


@pytest.mark.gpu
def test_predict_route_on_the_device_text_path():
    """The route around the device network: the page holds the texts the
    reference's tokenizer and the CPU checker produced (the GPT-NeoX fixture)."""
    from fastapi.testclient import TestClient

    import rustcrates_amd as ra
    from rustcrates_amd import configs
    from test_text import FIXTURE, MODEL, FixtureTokenizer

    loop = next(lp for lp in FIXTURE["text_loop"] if lp["inputs"][0].isascii() and len(lp["inputs"]) == 1)
    g = configs.build_network(ra.Network(0), MODEL)
    client = TestClient(server.create_app(server.device_predict_by_text(g, FixtureTokenizer())))
    r = client.post("/api/predict", data={"prompt": loop["inputs"][0]})
    print(f"/api/predict: {r.status_code}, {loop['texts'][0]!r}", flush=True)
    assert r.status_code == 200
    assert html.escape(str(loop["texts"])) in r.text
    g.close()
