"""Copy a selection of the reference's committed LightGBM v4 model texts.

Run in the build container (where /root/reference exists):

    python tests/golden/make_model_text_golden.py

The files are data of the reference's own tests (model texts written by the real
LightGBM 4.6 binary, crates/oracle-harness/tests/fixtures/**); they are copied
unchanged to tests/golden/model_text/<name>.txt.  Chosen to cover every envelope
and tree-block form the writer emits: monotone constraints, categorical bitsets
(num_cat > 0), a constant first tree (empty leaf_weight), average_output (random
forest), no objective line, multiclass / multiclassova, the exp-family and
cross-entropy objectives, DART shrinkage values, and the boosting spine models.
"""
import os
import shutil

FIX = "/root/reference/crates/oracle-harness/tests/fixtures"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_text")
FILES = {
    "mono_mixed": "constraints/mono_mixed.txt",
    "cat_manyvsmany": "categorical/cat_manyvsmany.txt",
    "cat_onehot": "categorical/cat_onehot.txt",
    "l1_constant_tree": "boosting/regression_l1_bag1_es0_bfa0_model.txt",
    "rf_multi_bag": "rf/rf_multi_bag_model.txt",
    "rf_single_bag": "rf/rf_single_bag_model.txt",
    "custom_no_objective": "boosting/custom_spine_model.txt",
    "multiclassova_spine": "boosting/multiclassova_spine_model.txt",
    "multiclass_spine": "boosting/multiclass_spine_model.txt",
    "poisson_spine": "boosting/poisson_spine_model.txt",
    "xentlambda_spine": "boosting/cross_entropy_lambda_spine_model.txt",
    "dart_u1_x1_bag1": "dart/dart_u1_x1_bag1_model.txt",
    "na_missing": "na_missing/model_real.txt",
    "binary_spine": "boosting/binary_spine_model.txt",
    "regression_spine": "boosting/regression_spine_model.txt",
    "forced_nested": "constraints/forced_nested.txt",
}


# The binary spine's per-iteration goldens (boosting_parity.rs:787-810): raw scores
# after every iteration (f64 bits), iteration-1 and iteration-5 gradients (f32 bits)
# and the transformed predictions (f64 bits) of the real binary on the 12-row corpus.
SPINE = ["binary_scores.txt", "binary_gh_iter1.txt", "binary_gh_iterN.txt",
         "binary_spine_pred.txt"]
# Prediction early stopping (predict_parity.rs:160-226): model, input rows (f64 bits)
# and the real binary's frozen raw scores per (freq, margin) cell.
PREDICT_MODES = {"numeric": ["model.txt", "X.txt", "early_stop.txt", "contrib.txt"],
                 "multiclass": ["model.txt", "X.txt", "early_stop.txt", "contrib.txt"],
                 "categorical": ["model.txt", "X.txt", "contrib.txt"]}


def main():
    os.makedirs(OUT, exist_ok=True)
    for name, rel in FILES.items():
        shutil.copyfile(os.path.join(FIX, rel), os.path.join(OUT, name + ".txt"))
        print(name, "<-", rel)
    os.makedirs(os.path.join(OUT, "spine"), exist_ok=True)
    for name in SPINE:
        shutil.copyfile(os.path.join(FIX, "boosting", name), os.path.join(OUT, "spine", name))
    for corpus, names in PREDICT_MODES.items():
        dst = os.path.join(os.path.dirname(OUT), "predict_modes", corpus)
        os.makedirs(dst, exist_ok=True)
        for name in names:
            shutil.copyfile(os.path.join(FIX, "predict_modes", corpus, name), os.path.join(dst, name))


if __name__ == "__main__":
    main()
