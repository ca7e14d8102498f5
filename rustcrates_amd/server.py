"""The reference's HTTP front of the greedy text loop (src/main.rs:65-87,
138-155): POST /api/predict with a urlencoded form field `prompt` runs
fix_encoding (utils/string.rs:3-7) and predict_by_text
(network_types/transformer/transformer_network.rs:638-660), and answers with
an HTML page holding the prompt and the predicted texts.

predict_by_text loads the model from its store for every call and runs
predict_token_by_token on it; here the model stays on the device and the text
loop (rustcrates_amd.text) resets its caches for every call, which is the same
state.  The training routes (/api/train, /api/train_status) and the page
template belong to the reference's application, not to the predict path, and
are not served.

    python -m rustcrates_amd.server --tokenizer gpt-neox-20b.json [--model net.bin --embeddings pairs.bin] [--port 7860]
"""
import argparse
import html
import urllib.parse

# WHATWG windows-1252 (encoding_rs, which fix_encoding calls): cp1252, with the
# five bytes cp1252 leaves undefined decoded to the C1 code points of equal value
_CP1252_GAPS = {0x81, 0x8D, 0x8F, 0x90, 0x9D}
_BYTE_TO_CHAR = [chr(b) if b < 0x80 or b in _CP1252_GAPS else bytes([b]).decode("cp1252") for b in range(256)]


def fix_encoding(s: str) -> str:
    """The UTF-8 bytes of s read as windows-1252 (utils/string.rs:3-7)."""
    return "".join(_BYTE_TO_CHAR[b] for b in s.encode("utf-8"))


def _page(prompt, result) -> str:
    out = "" if result is None else f"<p>{html.escape(str(result))}</p>"
    text = "" if prompt is None else html.escape(prompt)
    return ("<!doctype html><html><body><form method=\"post\" action=\"/api/predict\">"
            f"<textarea name=\"prompt\" required>{text}</textarea><button type=\"submit\">Predict</button></form>"
            f"{out}</body></html>")


def create_app(predict_by_text):
    """The routes, around predict_by_text(list of texts) -> list of texts."""
    from fastapi import FastAPI, Request
    from fastapi.responses import HTMLResponse

    app = FastAPI()

    @app.get("/", response_class=HTMLResponse)
    def index():
        return _page(None, None)

    @app.post("/api/predict", response_class=HTMLResponse)
    async def api_predict(request: Request):
        fields = urllib.parse.parse_qs((await request.body()).decode("utf-8"), keep_blank_values=True)
        if "prompt" not in fields:  # web::Form rejects a form without the field
            return HTMLResponse("missing field `prompt`", status_code=400)
        prompt = fields["prompt"][0]
        output = predict_by_text([fix_encoding(prompt)])
        return _page(prompt, output)

    return app


def device_predict_by_text(net, tokenizer):
    """predict_by_text on a device network: the texts of predict_token_by_token."""
    from . import text

    def run(inputs):
        return text.predict_token_by_token(net, inputs, tokenizer)[1]

    return run


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--tokenizer", required=True, help="the GPT-NeoX tokenizer JSON the reference loads")
    ap.add_argument("--model", help="a reference NeuralNetwork file (bincode); default: create_transformer's stack, seeded")
    ap.add_argument("--embeddings", help="the model's embedding (id, vector) pairs as model_io writes them")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--host", default="0.0.0.0")
    ap.add_argument("--port", type=int, default=7860)
    args = ap.parse_args(argv)
    import uvicorn

    from . import TRAINING, Network, configs, model_io, text

    net = Network(0)
    if args.model:
        with open(args.model, "rb") as f:
            model = model_io.read_network(f.read())
        pairs = None
        if args.embeddings:
            with open(args.embeddings, "rb") as f:
                pairs = model_io.read_embedding_pairs(f.read())
        model_io.to_device(model, net, pairs)
    else:  # predict_by_text's fallback when its store holds no model: create_transformer(TRAINING)
        configs.build_reference_default(net, seed=args.seed, mode=TRAINING)
    app = create_app(device_predict_by_text(net, text.load_tokenizer(args.tokenizer)))
    uvicorn.run(app, host=args.host, port=args.port)


if __name__ == "__main__":
    main()
